// Argument block of the paged decode kernels, passed by value.  Shared by the
// kernels (hipcc) and the host launcher (g++), so it holds only fixed-size
// C types.
#pragma once
#include <stdint.h>

struct luc_decode_args {
  uint16_t* q;              // row b at q + b*q_stride; q-head j at + j*head_dim
  const uint16_t* q_bias;   // step kernel: [Hq*head_dim] or null
  uint16_t* k_new;          // step kernel: row b at k_new + b*q_stride, [Hkv*head_dim]
  const uint16_t* k_bias;   // step kernel: [Hkv*head_dim] or null
  const uint16_t* v_new;    // step kernel: row b at v_new + b*q_stride, [Hkv*head_dim]
  const uint16_t* v_bias;   // step kernel: [Hkv*head_dim] or null
  const float* cos_t;       // step kernel: [max_pos][head_dim/2]
  const float* sin_t;
  int64_t q_stride;
  uint16_t* k_pool;         // [blocks][num_layers][Hkv][16][head_dim]
  uint16_t* v_pool;
  const int32_t* tables;    // [batch][table_stride]
  int64_t table_stride;
  const int32_t* positions; // [batch]
  int32_t batch, layer, num_layers, hkv;
  int32_t num_blocks;       // pages per pool: table entries outside [0, num_blocks) are never used
  float qk_scale_log2;      // sm_scale * log2(e)
  int32_t max_ctx, split_tokens, max_splits;
  float* ws_ml;             // [batch*Hkv][max_splits][G][2]  (max, sum) per split
  float* ws_o;              // [batch*Hkv][max_splits][G*head_dim]
  int32_t* ws_cnt;          // [batch*Hkv] split arrivals, zero between launches
  uint16_t* out;            // row b at out + b*out_stride, [Hq*head_dim]
  int64_t out_stride;
};
