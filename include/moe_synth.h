/*
 * moe_synth.h -- seeded synthetic workloads for the MoE block (host side).
 *
 * No counterpart in the reference (its tree holds no data files: data/ and
 * model.bin are absent).  The benchmarks and tests fill weights and
 * activations with these generators so that every process, on any host,
 * produces bit-identical inputs from (seed, stream, index):
 *
 *   value i of stream s = std * Box-Muller normal from two 53-bit uniforms
 *                         drawn by a SplitMix64-style counter hash.
 *
 * Stream numbering follows a fixed draw order: gate = 0, bias = 1, then for
 * expert e: w1 = 2+3e, w3 = 3+3e, w2 = 4+3e, and x = 2+3E.
 */
#ifndef MOE_SYNTH_H
#define MOE_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] = std * N(0,1) sample i of (seed, stream), for i in [first, first+n).
 * Multi-threaded over host cores; results do not depend on the thread count. */
void moe_synth_normal(uint64_t seed, uint64_t stream, float std_dev,
                      uint64_t first, float *out, size_t n);

/* Stream id helpers for the draw order above. */
uint64_t moe_synth_stream_gate(void);
uint64_t moe_synth_stream_bias(void);
uint64_t moe_synth_stream_w1(int expert);
uint64_t moe_synth_stream_w3(int expert);
uint64_t moe_synth_stream_w2(int expert);
uint64_t moe_synth_stream_x(int num_experts);

/* Threads used by moe_synth_normal (<=0: hardware concurrency, max 16). */
void moe_synth_set_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
