// Gated delta rule, token-recurrent form, with the block-causal canvas readout.
//
// Per value head h and row t (g = log decay, scale applied to q):
//   S = e^{g_t} S;  kv = S k_t;  delta = beta_t (v_t - kv);  S += delta k_t^T;  o_t = S q_t
// causal_mode 1: every row reads its own state. causal_mode 2: rows t < num_clean read their own
// state, rows t >= num_clean read the block-end state (the state after all T rows).
// Block-bidirectional readout (trida_gdr_block_bidir): per block of `bidir` rows, a backward sub-scan
// over the block's rows in reverse from the block-entry state, then the causal forward sub-scan; each
// row reads out the mean of the two; the state carried on is the forward one.
//
// Launch: block = (sequence b, value head h, v-tile). Each wave owns 4 value columns; the 16 lanes of
// a column each hold KPL = Dk/16 consecutive k entries of that column's state in registers, so the
// two dot products of a step reduce over one 16-lane DPP row (no LDS round trip). The rows of q, k,
// v, g, beta are staged through LDS 32 at a time (all loads of a chunk in flight together).
// Critical path per step: decay, two independent dots (S'k and S'q), two interleaved row reductions,
// then o = S'q + delta (k.q); the state update itself is off the path.
#include "common.h"

namespace trida {
namespace {

constexpr int kLanesPerV = 16;
constexpr int kVPerWave = kWave / kLanesPerV;  // 4
constexpr int kTC = 64;                        // rows staged per LDS chunk (a canvas block fits in one)

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}
// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  return v;
}
__device__ __forceinline__ void row16_sum2(float& a, float& b) {
  a += dpp<0x128>(a);
  b += dpp<0x128>(b);
  a += dpp<0x124>(a);
  b += dpp<0x124>(b);
  a += dpp<0x4E>(a);
  b += dpp<0x4E>(b);
  a += dpp<0xB1>(a);
  b += dpp<0xB1>(b);
}

struct RecArgs {
  const uint16_t* q;  // [B, T, Hk, Dk]
  const uint16_t* k;
  const uint16_t* v;  // [B, T, Hv, Dv]
  const float* g;     // [B, T, Hv]
  const float* beta;
  const float* state_in;  // [B, Hv, Dv, Dk]
  uint16_t* out;          // [B, T, Hv, Dv]
  float* state_out;
  float* state_clean;
  int T, Hk, Hv, Dk, Dv;
  int causal_mode, num_clean;
  float scale;
  int bidir;  // > 0: block-bidirectional readout over blocks of this many rows (causal_mode 1)
};

template <int KPL, int NW>
__global__ __launch_bounds__(NW* kWave) void gdr_recurrent_kernel(RecArgs a) {
  constexpr int Dk = KPL * kLanesPerV;
  constexpr int VPB = NW * kVPerWave;
  const int tiles = a.Dv / VPB;
  const int vt = blockIdx.x % tiles;
  const int h = (blockIdx.x / tiles) % a.Hv;
  const int b = blockIdx.x / (tiles * a.Hv);
  const int hk = h / (a.Hv / a.Hk);
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int vl = wave * kVPerWave + lane / kLanesPerV;  // value column within the tile
  const int v = vt * VPB + vl;
  const int kl = lane % kLanesPerV;                      // k slice [kl*KPL, kl*KPL+KPL)

  __shared__ __align__(16) uint16_t s_q[kTC][Dk];
  __shared__ __align__(16) uint16_t s_k[kTC][Dk];
  __shared__ float s_v[kTC][VPB];
  __shared__ float s_g[kTC], s_b[kTC];
  __shared__ float s_ob[kTC][VPB];  // backward sub-scan outputs of the block-bidirectional readout

  const int64_t st_off = (((int64_t)b * a.Hv + h) * a.Dv + v) * Dk + kl * KPL;
  float s[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) s[i] = a.state_in[st_off + i];

  const int nc = a.causal_mode == 2 ? min(a.num_clean, a.T) : a.T;
  const int64_t qk_row = (int64_t)a.Hk * Dk;  // elements between rows t and t+1
  const uint16_t* qb = a.q + (int64_t)b * a.T * qk_row + (int64_t)hk * Dk;
  const uint16_t* kb = a.k + (int64_t)b * a.T * qk_row + (int64_t)hk * Dk;
  const int64_t v_row = (int64_t)a.Hv * a.Dv;
  const uint16_t* vb = a.v + (int64_t)b * a.T * v_row + (int64_t)h * a.Dv + vt * VPB;
  uint16_t* ob = a.out + (int64_t)b * a.T * v_row + (int64_t)h * a.Dv + v;
  const float* gb = a.g + (int64_t)b * a.T * a.Hv + h;
  const float* bb = a.beta + (int64_t)b * a.T * a.Hv + h;

  // rows staged per chunk: whole blocks when the readout is block-bidirectional
  const int tcn = a.bidir > 0 ? (kTC / a.bidir) * a.bidir : kTC;
  // one step of the recurrence on state st with staged row r; returns the row's readout S'q
  auto step = [&](float (&st)[KPL], int r) -> float {
    float kk[KPL], qq[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      kk[i] = bf2f(s_k[r][kl * KPL + i]);
      qq[i] = bf2f(s_q[r][kl * KPL + i]) * a.scale;
    }
    const float eg = s_g[r];
    float kv = 0.f, sq = 0.f, kq = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      st[i] *= eg;
      kv = fmaf(st[i], kk[i], kv);
      sq = fmaf(st[i], qq[i], sq);
      kq = fmaf(kk[i], qq[i], kq);
    }
    row16_sum2(kv, sq);
    kq = row16_sum(kq);
    const float delta = (s_v[r][vl] - kv) * s_b[r];
#pragma unroll
    for (int i = 0; i < KPL; ++i) st[i] = fmaf(kk[i], delta, st[i]);
    return fmaf(delta, kq, sq);
  };
  for (int t0 = 0; t0 < a.T; t0 += tcn) {
    const int tn = min(tcn, a.T - t0);
    __syncthreads();  // previous chunk fully consumed
    // stage q, k rows (16-byte pieces), v tile, g, beta
    constexpr int kPieces = Dk / 8;
    for (int p = tid; p < tn * kPieces; p += NW * kWave) {
      const int r = p / kPieces, c = (p % kPieces) * 8;
      *reinterpret_cast<u32x4*>(&s_q[r][c]) = *reinterpret_cast<const u32x4*>(qb + (int64_t)(t0 + r) * qk_row + c);
      *reinterpret_cast<u32x4*>(&s_k[r][c]) = *reinterpret_cast<const u32x4*>(kb + (int64_t)(t0 + r) * qk_row + c);
    }
    for (int p = tid; p < tn * VPB; p += NW * kWave) {
      const int r = p / VPB, c = p % VPB;
      s_v[r][c] = bf2f(vb[(int64_t)(t0 + r) * v_row + c]);
    }
    for (int p = tid; p < tn; p += NW * kWave) {
      s_g[p] = __expf(gb[(int64_t)(t0 + p) * a.Hv]);
      s_b[p] = bb[(int64_t)(t0 + p) * a.Hv];
    }
    __syncthreads();

    if (a.bidir > 0) {
      // each block: a backward sub-scan from the block-entry state (a register copy), then the causal
      // forward sub-scan; a row reads out the mean of the two
      for (int r0 = 0; r0 < tn; r0 += a.bidir) {
        const int r1 = min(r0 + a.bidir, tn);
        float sb[KPL];
#pragma unroll
        for (int i = 0; i < KPL; ++i) sb[i] = s[i];
        for (int r = r1 - 1; r >= r0; --r) {
          const float o = step(sb, r);
          if (kl == 0) s_ob[r][vl] = o;
        }
        for (int r = r0; r < r1; ++r) {
          const float o = step(s, r);
          if (kl == 0) ob[(int64_t)(t0 + r) * v_row] = f2bf(0.5f * (o + s_ob[r][vl]));
        }
      }
      continue;
    }
#pragma unroll 2
    for (int r = 0; r < tn; ++r) {
      const int t = t0 + r;
      const float o = step(s, r);
      if (t < nc && kl == 0) ob[(int64_t)t * v_row] = f2bf(o);
      if (t == nc - 1 && a.state_clean) {
#pragma unroll
        for (int i = 0; i < KPL; ++i) a.state_clean[st_off + i] = s[i];
      }
    }
  }
  if (nc == 0 && a.state_clean) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) a.state_clean[st_off + i] = a.state_in[st_off + i];
  }
  // MASK rows (causal_mode 2): read the block-end state
  for (int t = nc; t < a.T; ++t) {
    const u32x4* qp = reinterpret_cast<const u32x4*>(qb + (int64_t)t * qk_row + kl * KPL);
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; i += 8) {
      const u32x4 w = qp[i / 8];
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4 && i + 2 * j < KPL; ++j) {
        o = fmaf(s[i + 2 * j], bf2f((uint16_t)(ws[j] & 0xffff)) * a.scale, o);
        o = fmaf(s[i + 2 * j + 1], bf2f((uint16_t)(ws[j] >> 16)) * a.scale, o);
      }
    }
    o = row16_sum(o);
    if (kl == 0) ob[(int64_t)t * v_row] = f2bf(o);
  }
  if (a.state_out) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) a.state_out[st_off + i] = s[i];
  }
}

template <int KPL>
int launch_kpl(const RecArgs& a, int B, hipStream_t st) {
  // widest block whose v-tile divides Dv; more, narrower blocks when the grid would be small
  int nw = 4;
  while (nw > 1 && (a.Dv % (nw * kVPerWave) != 0 || (int64_t)B * a.Hv * (a.Dv / (nw * kVPerWave)) < 256)) nw /= 2;
  if (a.Dv % (nw * kVPerWave) != 0) return TRIDA_ERR_ARG;
  const unsigned grid = (unsigned)((int64_t)B * a.Hv * (a.Dv / (nw * kVPerWave)));
  switch (nw) {
    case 4: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 4>), dim3(grid), dim3(4 * kWave), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 2>), dim3(grid), dim3(2 * kWave), 0, st, a); break;
    default: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 1>), dim3(grid), dim3(kWave), 0, st, a); break;
  }
  return launch_status("gdr_recurrent");
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_gdr_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                   const float* beta, const float* state_in, uint16_t* out, float* state_out,
                                   float* state_clean, int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                                   int64_t Dk, int64_t Dv, int causal_mode, int64_t num_clean, float scale,
                                   void* stream) {
  TRIDA_CHECK(q && k && v && g && beta && state_in && out, TRIDA_ERR_NULL,
              "gdr_recurrent: q, k, v, g, beta, state_in and out are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, TRIDA_ERR_ARG,
              "gdr_recurrent: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld", (long long)B, (long long)T,
              (long long)Hk, (long long)Hv);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128 || Dk == 256, TRIDA_ERR_ARG,
              "gdr_recurrent: Dk must be 32, 64, 128 or 256 (got %lld)", (long long)Dk);
  TRIDA_CHECK(Dv > 0 && Dv % 4 == 0, TRIDA_ERR_ARG, "gdr_recurrent: Dv must be a multiple of 4");
  TRIDA_CHECK(causal_mode == 1 || causal_mode == 2, TRIDA_ERR_ARG, "gdr_recurrent: causal_mode is 1 or 2");
  TRIDA_CHECK(num_clean >= 0, TRIDA_ERR_ARG, "gdr_recurrent: num_clean >= 0");
  TRIDA_CHECK(state_clean == nullptr || (state_clean != state_in && state_clean != state_out), TRIDA_ERR_ARG,
              "gdr_recurrent: state_clean must not alias state_in or state_out");
  TRIDA_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0, TRIDA_ERR_ALIGN,
              "gdr_recurrent: q and k must be 16-byte aligned");
  TRIDA_CHECK(B * T * Hv < INT32_MAX, TRIDA_ERR_ARG, "gdr_recurrent: problem too large");
  RecArgs a{q, k, v, g, beta, state_in, out, state_out, state_clean, (int)T, (int)Hk, (int)Hv, (int)Dk,
            (int)Dv, causal_mode, (int)num_clean, scale, 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2>(a, (int)B, st);
    case 64: return launch_kpl<4>(a, (int)B, st);
    case 128: return launch_kpl<8>(a, (int)B, st);
    default: return launch_kpl<16>(a, (int)B, st);
  }
}

extern "C" int trida_gdr_block_bidir(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                     const float* beta, const float* state_in, uint16_t* out, float* state_out,
                                     int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                                     int64_t block_size, float scale, void* stream) {
  TRIDA_CHECK(q && k && v && g && beta && state_in && out, TRIDA_ERR_NULL,
              "gdr_block_bidir: q, k, v, g, beta, state_in and out are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, TRIDA_ERR_ARG, "gdr_block_bidir: bad sizes");
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128 || Dk == 256, TRIDA_ERR_ARG,
              "gdr_block_bidir: Dk must be 32, 64, 128 or 256 (got %lld)", (long long)Dk);
  TRIDA_CHECK(Dv > 0 && Dv % 4 == 0, TRIDA_ERR_ARG, "gdr_block_bidir: Dv must be a multiple of 4");
  TRIDA_CHECK(block_size >= 1 && block_size <= kTC, TRIDA_ERR_ARG, "gdr_block_bidir: block_size in [1, %d]", kTC);
  TRIDA_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0, TRIDA_ERR_ALIGN,
              "gdr_block_bidir: q and k must be 16-byte aligned");
  TRIDA_CHECK(B * T * Hv < INT32_MAX, TRIDA_ERR_ARG, "gdr_block_bidir: problem too large");
  RecArgs a{q, k, v, g, beta, state_in, out, state_out, nullptr, (int)T, (int)Hk, (int)Hv, (int)Dk,
            (int)Dv, 1, (int)T, scale, (int)block_size};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2>(a, (int)B, st);
    case 64: return launch_kpl<4>(a, (int)B, st);
    case 128: return launch_kpl<8>(a, (int)B, st);
    default: return launch_kpl<16>(a, (int)B, st);
  }
}
