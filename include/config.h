// Model and MoE constants of the LFM2-8B-A1B-style decoder the MoE block
// belongs to.  Values and names follow reference include/config.h:4-20; only
// the ones this MoE build uses are kept (the pipeline, attention-tile and fp16
// settings of config.h:22-56 belong to parts of the reference that are out of
// scope here).
#pragma once

#include <cstddef>

constexpr size_t VOCAB_SIZE = 65536;
constexpr size_t HIDDEN_SIZE = 2048;
constexpr size_t INTERMEDIATE_SIZE = 7168;
constexpr size_t NUM_HIDDEN_LAYERS = 24;
constexpr float RMS_NORM_EPS = 1e-5f;

constexpr size_t NUM_EXPERTS = 32;
constexpr size_t NUM_EXPERTS_PER_TOK = 4;
constexpr size_t NUM_DENSE_LAYERS = 2;
constexpr size_t MOE_INTERMEDIATE_SIZE = 1792;
constexpr float ROUTED_SCALING_FACTOR = 1.0f;
constexpr bool NORM_TOPK_PROB = true;
constexpr bool USE_EXPERT_BIAS = true;

// Scratch capacity of a SparseMoeBlock (tokens per forward).  The reference
// hard-codes 4096 (layer.cu:1399); 16384 covers the skewed-routing workload.
constexpr int MOE_DEFAULT_MAX_TOKENS = 16384;
