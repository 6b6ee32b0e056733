// The chunked gated delta rule over a long prefix (gdn_prefix.hip: a chunk-parallel preparation, then the
// scan), dispatched by trida_gdr_chunk.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trida {

struct PrefixArgs {
  const uint16_t* q;      // [B, T, Hk, 128] bf16 (read with out only)
  const uint16_t* k;      // [B, T, Hk, 128] bf16
  const uint16_t* v;      // [B, T, Hv, Dv] bf16
  const float* g;         // [B, T, Hv] log decay
  const float* beta;      // [B, T, Hv]
  const float* state_in;  // [B, Hv, Dv, 128] fp32
  uint16_t* out;          // [B, T, Hv, Dv] bf16 or null
  float* state_out;       // [B, Hv, Dv, 128] fp32 or null (the state after all T rows)
  void* ws;               // kPrefixWsBytes per (sequence, chunk, value head), 16-byte aligned
  int T, Hk, Hv, Dv, nchunks;
  float scale;
};

// workspace bytes per (sequence, 64-row chunk, value head): T (bf16 hi + lo) and M (bf16) fragments, the
// chunk's decays (fp32)
constexpr int64_t kPrefixWsBytes = 19456;

// T > 64, Dk == 128, Dv % 16 == 0, at most 256 workgroups (B * Hv * Dv / 16); every row causal, the state
// after the last row
bool gdr_prefix_supported(int64_t B, int64_t T, int64_t Hv, int64_t Dk, int64_t Dv);
int gdr_prefix_launch(const PrefixArgs& a, int64_t B, hipStream_t stream);

}  // namespace trida
