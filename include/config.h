// Model constants of the LFM2-8B-A1B-style decoder (reference
// include/config.h:4-31, same names and values).  The pipeline, tile and
// fp16 settings of config.h:33-56 belong to the reference's CUDA kernels and
// its 4-GPU pipeline, which this build replaces.
#pragma once

#include <cstddef>

constexpr size_t VOCAB_SIZE = 65536;
constexpr size_t HIDDEN_SIZE = 2048;
constexpr size_t INTERMEDIATE_SIZE = 7168;
constexpr size_t NUM_HIDDEN_LAYERS = 24;
constexpr size_t NUM_ATTENTION_HEADS = 32;
constexpr size_t NUM_KEY_VALUE_HEADS = 8;
constexpr size_t MAX_POSITION_EMBEDDINGS = 128000;
constexpr float RMS_NORM_EPS = 1e-5f;
constexpr float ROPE_THETA = 1000000.0f;

constexpr size_t NUM_EXPERTS = 32;
constexpr size_t NUM_EXPERTS_PER_TOK = 4;
constexpr size_t NUM_DENSE_LAYERS = 2;
constexpr size_t MOE_INTERMEDIATE_SIZE = 1792;
constexpr float ROUTED_SCALING_FACTOR = 1.0f;
constexpr bool NORM_TOPK_PROB = true;
constexpr bool USE_EXPERT_BIAS = true;

constexpr size_t CONV_L_CACHE = 3;
constexpr bool USE_CONV_BIAS = false;

constexpr bool ATTENTION_BIAS = false;
constexpr size_t HEAD_DIM = HIDDEN_SIZE / NUM_ATTENTION_HEADS;
constexpr size_t NUM_KEY_VALUE_GROUPS = NUM_ATTENTION_HEADS / NUM_KEY_VALUE_HEADS;
constexpr size_t CONV_KERNEL = CONV_L_CACHE;

// 0 = attention layer, 1 = short-conv layer
constexpr int LAYER_TYPES[] = {1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 0, 1, 1};

// Scratch capacity of a SparseMoeBlock (tokens per forward).  The reference
// hard-codes 4096 (layer.cu:1399); 16384 covers the skewed-routing workload.
constexpr int MOE_DEFAULT_MAX_TOKENS = 16384;
