// The single-block MFMA readout of the gated delta rule (gdn_block.hip), dispatched by trida_gdr_chunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trida {

struct BlockArgs {
  const uint16_t* q;      // [B, T, Hk, 128] bf16
  const uint16_t* k;      // [B, T, Hk, 128] bf16
  const uint16_t* v;      // [B, T, Hv, Dv] bf16
  const float* g;         // [B, T, Hv] log decay
  const float* beta;      // [B, T, Hv]
  const float* state;     // [B, Hv, Dv, 128] fp32, read only
  uint16_t* out;          // [B, T, Hv, Dv] bf16
  int T, Hk, Hv, Dv;
  int causal_mode;        // 1: every row causal; 2: rows >= num_clean read the block-end state
  int num_clean;          // clamped to [0, T]
  float scale;
};

// T in [1, 64], Dk == 128, Dv % 128 == 0
bool gdr_block_supported(int64_t T, int64_t Dk, int64_t Dv);
int gdr_block_launch(const BlockArgs& a, int64_t B, hipStream_t stream);

}  // namespace trida
