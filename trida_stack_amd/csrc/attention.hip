// Canvas attention over a bf16 KV cache (draft / verify / mixed masks), MFMA on gfx950.
//
// Query rows of one KV head are the pairs (canvas row t, GQA head g), row m = t * G + g, so the G query
// heads sharing a KV head form one [T*G, D] matrix. Keys p in [0, prefix + T) of the cache; row t sees
// key p when p < prefix (the committed prefix) or, inside the block (j = p - prefix):
//   mask 0 (verify, causal)       j <= t
//   mask 1 (draft, bidirectional) always
//   mask 2 (canvas, mixed)        j <= t for t < n_clean, always for t >= n_clean
//
// attn_partial: workgroup = (sequence, KV head, query tile of <= 144 rows, key split), 4 waves.
//   Per block of 64 keys: each wave computes S = Q K^T for its 16 keys and all rows of the tile with
//   v_mfma_f32_16x16x32_bf16 (K fragments straight from global memory into registers, Q from LDS),
//   the online-softmax statistics are combined across the 4 waves through LDS, P is written to LDS in
//   bf16, and each wave accumulates O[:, its D/4 columns] += P V with V staged transposed in LDS.
//   Writes the unnormalised O, row max and row sum of its split.
// attn_combine: merges the splits per row (log-sum-exp weights), applies the optional output gate
//   sigmoid(gate) and writes bf16.
#include <math.h>

#include "common.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kNW = 4;
constexpr int kMT = 144;        // query rows per workgroup (9 MFMA row tiles)
constexpr int kRT = kMT / 16;
constexpr int kKB = 64;         // keys per block
constexpr int kKP = kKB + 8;    // padded LDS row of P / V^T (elements)
constexpr float kLog2e = 1.4426950408889634f;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0x128>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0xB1>(v));
  return v;
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0x128>(v);
  v += dpp<0x124>(v);
  v += dpp<0x4E>(v);
  v += dpp<0xB1>(v);
  return v;
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

struct AttnArgs {
  const uint16_t* q;        // [B, T, Hq, D]
  const uint16_t* k_cache;  // [B, Hkv, Lmax, D]
  const uint16_t* v_cache;
  const int32_t* prefix;    // [B]
  float* opart;             // [B, Hkv, QT, S, kMT, D]
  float* mpart;             // [B, Hkv, QT, S, kMT]
  float* lpart;
  int T, Hq, Hkv, G, Lmax, S, QT, mask_mode, n_clean;
  float scale_log2;         // softmax scale * log2(e)
};

__device__ __forceinline__ bool visible(int p, int prefix, int t, int mode, int n_clean) {
  const int j = p - prefix;
  if (j < 0) return true;
  if (mode == 1) return true;
  if (mode == 2 && t >= n_clean) return true;
  return j <= t;
}

template <int D>
__global__ __launch_bounds__(kNW* kWave) void attn_partial_kernel(AttnArgs a) {
  constexpr int DP = D + 8;       // padded LDS row of Q (elements)
  constexpr int KC = D / 32;      // MFMA k-chunks over the head dim
  constexpr int CPW = D / kNW;    // O columns per wave
  constexpr int CT = CPW / 16;    // O column tiles per wave
  __shared__ __align__(16) uint16_t sQ[kMT * DP];
  __shared__ __align__(16) uint16_t sVt[D * kKP];
  __shared__ __align__(16) uint16_t sP[kMT * kKP];
  __shared__ float sMax[kNW][kMT], sSum[kNW][kMT];
  __shared__ float sM[kMT], sL[kMT];

  int idx = blockIdx.x;
  const int s = idx % a.S;
  idx /= a.S;
  const int qt = idx % a.QT;
  idx /= a.QT;
  const int hk = idx % a.Hkv;
  const int b = idx / a.Hkv;
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int M = a.T * a.G;
  const int m0 = qt * kMT;
  const int rows = min(kMT, M - m0);
  const int prefix = a.prefix[b];
  const int nk = prefix + a.T;
  // key range of this split: whole blocks of 64
  const int nblk = (nk + kKB - 1) / kKB;
  const int bps = (nblk + a.S - 1) / a.S;
  const int kb0 = s * bps, kb1 = min(nblk, kb0 + bps);
  // the last query row of the tile bounds the keys any row can see under the causal masks
  const int t_last = (m0 + rows - 1) / a.G;
  const int kmax = (a.mask_mode == 1 || (a.mask_mode == 2 && t_last >= a.n_clean)) ? nk : min(nk, prefix + t_last + 1);

  const int64_t pbase = ((((int64_t)b * a.Hkv + hk) * a.QT + qt) * a.S + s);
  if (kb0 >= kb1 || kb0 * kKB >= kmax) {
    // no key of this split is visible to the tile: only the (empty) row stats are written and the
    // combine skips the split without reading its O
    for (int r = tid; r < rows; r += kNW * kWave) {
      a.mpart[pbase * kMT + r] = -INFINITY;
      a.lpart[pbase * kMT + r] = 0.f;
    }
    return;
  }
  // ---- stage Q rows (zero padding rows) and init running stats
  for (int p = tid; p < kMT * (D / 8); p += kNW * kWave) {
    const int r = p / (D / 8), c = (p % (D / 8)) * 8;
    u32x4 val = {0u, 0u, 0u, 0u};
    if (r < rows) {
      const int m = m0 + r, t = m / a.G, g = m % a.G;
      val = *reinterpret_cast<const u32x4*>(a.q + (((int64_t)b * a.T + t) * a.Hq + hk * a.G + g) * D + c);
    }
    *reinterpret_cast<u32x4*>(&sQ[r * DP + c]) = val;
  }
  for (int r = tid; r < kMT; r += kNW * kWave) {
    sM[r] = -INFINITY;
    sL[r] = 0.f;
  }
  f32x4 o[kRT][CT];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint16_t* kh = a.k_cache + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;
  const uint16_t* vh = a.v_cache + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;

  for (int kb = kb0; kb < kb1 && kb * kKB < kmax; ++kb) {
    const int key0 = kb * kKB;
    __syncthreads();  // previous block's P / V^T fully consumed (and Q / stats staged)
    // ---- K fragments for this wave's 16 keys: B operand, col = key (l % 16), k = head dim
    const int my_key = key0 + w * 16 + (l % 16);
    const int kclamp = min(my_key, nk - 1);
    u32x4 kf[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      kf[kc] = *reinterpret_cast<const u32x4*>(kh + (int64_t)kclamp * D + kc * 32 + (l / 16) * 8);
    // ---- V block transposed into LDS: each thread moves one 8 keys x 8 columns square
    for (int p = tid; p < (kKB / 8) * (D / 8); p += kNW * kWave) {
      const int kg = p / (D / 8), cg = (p % (D / 8)) * 8;
      u32x4 rowv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int key = min(key0 + kg * 8 + j, nk - 1);
        rowv[j] = *reinterpret_cast<const u32x4*>(vh + (int64_t)key * D + cg);
      }
      const uint32_t* rw = reinterpret_cast<const uint32_t*>(rowv);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        // column c of the square: element c of each of the 8 key rows
        uint32_t e[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const uint32_t word = rw[j * 4 + c / 2];
          e[j] = (c & 1) ? (word >> 16) : (word & 0xffffu);
        }
        u32x4 packed;
        packed.x = e[0] | (e[1] << 16);
        packed.y = e[2] | (e[3] << 16);
        packed.z = e[4] | (e[5] << 16);
        packed.w = e[6] | (e[7] << 16);
        *reinterpret_cast<u32x4*>(&sVt[(cg + c) * kKP + kg * 8]) = packed;
      }
    }
    // ---- S = Q K^T for this wave's 16 keys, all row tiles; mask; per-row block max
    float sv[kRT][4];
    const bool key_ok = my_key < nk;
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const u32x4 af = *reinterpret_cast<const u32x4*>(&sQ[(rt * 16 + (l % 16)) * DP + kc * 32 + (l / 16) * 8]);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(af), as_bf16x8(kf[kc]), c, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rt * 16 + (l / 16) * 4 + i;  // row within the tile
        const int t = (m0 + r) / a.G;
        const bool ok = key_ok && r < rows && visible(my_key, prefix, t, a.mask_mode, a.n_clean);
        sv[rt][i] = ok ? c[i] * a.scale_log2 : -INFINITY;
      }
    }
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float mx = row16_max(sv[rt][i]);
        if ((l % 16) == 0) sMax[w][rt * 16 + (l / 16) * 4 + i] = mx;
      }
    __syncthreads();
    // ---- P = exp2(S - m_new) (bf16 to LDS), partial row sums, rescale factors
    float alpha[kRT][4];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rt * 16 + (l / 16) * 4 + i;
        const float m_old = sM[r];
        float bm = sMax[0][r];
#pragma unroll
        for (int ww = 1; ww < kNW; ++ww) bm = fmaxf(bm, sMax[ww][r]);
        const float m_new = fmaxf(m_old, bm);
        const float m_use = m_new == -INFINITY ? 0.f : m_new;
        alpha[rt][i] = exp2f(m_old - m_use);
        const float p = exp2f(sv[rt][i] - m_use);
        sP[r * kKP + w * 16 + (l % 16)] = f2bf(p);
        const float ps = row16_sum(p);
        if ((l % 16) == 0) sSum[w][r] = ps;
      }
    __syncthreads();
    // ---- running stats (one thread per row) and O rescale
    for (int r = tid; r < kMT; r += kNW * kWave) {
      const float m_old = sM[r];
      float bm = sMax[0][r], ps = sSum[0][r];
#pragma unroll
      for (int ww = 1; ww < kNW; ++ww) {
        bm = fmaxf(bm, sMax[ww][r]);
        ps += sSum[ww][r];
      }
      const float m_new = fmaxf(m_old, bm);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      sL[r] = sL[r] * exp2f(m_old - m_use) + ps;
      sM[r] = m_new;
    }
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[rt][ct][i] *= alpha[rt][i];
    // ---- O[:, wave columns] += P V: A = P (rows x keys), B = V^T fragment (col, 8 keys)
#pragma unroll
    for (int kk = 0; kk < kKB / 32; ++kk) {
      bf16x8 bfr[CT];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        bfr[ct] = as_bf16x8(*reinterpret_cast<const u32x4*>(
            &sVt[(w * CPW + ct * 16 + (l % 16)) * kKP + kk * 32 + (l / 16) * 8]));
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const bf16x8 af = as_bf16x8(*reinterpret_cast<const u32x4*>(&sP[(rt * 16 + (l % 16)) * kKP + kk * 32 + (l / 16) * 8]));
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[ct], o[rt][ct], 0, 0, 0);
      }
    }
  }
  __syncthreads();
  // ---- write this split's unnormalised O and row stats (fp32)
  float* op = a.opart + pbase * kMT * D;
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = rt * 16 + (l / 16) * 4 + i;
        if (r < rows) op[(int64_t)r * D + w * CPW + ct * 16 + (l % 16)] = o[rt][ct][i];
      }
  for (int r = tid; r < rows; r += kNW * kWave) {
    a.mpart[pbase * kMT + r] = sM[r];
    a.lpart[pbase * kMT + r] = sL[r];
  }
}

struct CombineArgs {
  const float* opart;
  const float* mpart;
  const float* lpart;
  const uint16_t* gate;  // row t, head h, dim d at gate + t * gate_st + h * gate_hs + d; or null
  uint16_t* out;         // [B, T, Hq, D]
  int T, Hq, Hkv, G, D, S, QT;
  int64_t gate_st, gate_hs;
};

// Block = a group of RB rows of one (sequence, KV head); thread = (row, 8 output columns). The split
// weights exp2(m_s - max) / sum of the group's rows are computed once into LDS; each thread then sums
// the O rows of the non-empty splits.
constexpr int kMaxSplits = 256;

__global__ __launch_bounds__(256) void attn_combine_kernel(CombineArgs a) {
  __shared__ float s_w[32][kMaxSplits];  // rows of the group x listed splits
  __shared__ float s_inv[32];
  __shared__ int s_list[kMaxSplits];
  __shared__ int s_cnt[4];
  const int M = a.T * a.G;
  const int per_row = a.D / 8;
  const int rb = 256 / per_row;  // rows per block: 8 (D=256), 16 (D=128), 32 (D=64)
  const int b = blockIdx.y / a.Hkv, hk = blockIdx.y % a.Hkv;
  const int m0 = blockIdx.x * rb;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  // list, in split order, the splits with a visible key for some row of the group (one split per
  // thread, S <= 256; wave ballots give each listed split its position)
  bool any = false;
  if (tid < a.S) {
    for (int i = 0; i < rb && m0 + i < M; ++i) {
      const int m = m0 + i;
      const int64_t bs = (((int64_t)b * a.Hkv + hk) * a.QT + m / kMT) * a.S;
      any |= a.mpart[(bs + tid) * kMT + m % kMT] != -INFINITY;
    }
  }
  const unsigned long long mask = __ballot(any);
  if (lane == 0) s_cnt[wave] = __popcll(mask);
  __syncthreads();
  int off = 0;
  for (int w = 0; w < wave; ++w) off += s_cnt[w];
  if (any) s_list[off + __popcll(mask & ((1ull << lane) - 1ull))] = tid;
  const int ns = s_cnt[0] + s_cnt[1] + s_cnt[2] + s_cnt[3];
  __syncthreads();
  // per row: max, weights and 1 / sum
  if (tid < rb && m0 + tid < M) {
    const int m = m0 + tid;
    const int64_t bs = (((int64_t)b * a.Hkv + hk) * a.QT + m / kMT) * a.S;
    const int r = m % kMT;
    float mx = -INFINITY;
    for (int j = 0; j < ns; ++j) mx = fmaxf(mx, a.mpart[(bs + s_list[j]) * kMT + r]);
    const float m_use = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f;
    for (int j = 0; j < ns; ++j) {
      const float w = exp2f(a.mpart[(bs + s_list[j]) * kMT + r] - m_use);
      s_w[tid][j] = w;
      lsum += w * a.lpart[(bs + s_list[j]) * kMT + r];
    }
    s_inv[tid] = lsum > 0.f ? 1.f / lsum : 0.f;
  }
  __syncthreads();
  const int i = tid / per_row;
  const int m = m0 + i;
  if (i >= rb || m >= M) return;
  const int c = (tid % per_row) * 8;
  const int64_t bs = (((int64_t)b * a.Hkv + hk) * a.QT + m / kMT) * a.S;
  const int r = m % kMT;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int j = 0; j < ns; ++j) {
    const float wgt = s_w[i][j];
    const f32x4* op = reinterpret_cast<const f32x4*>(a.opart + ((bs + s_list[j]) * kMT + r) * a.D + c);
    const f32x4 x0 = op[0], x1 = op[1];
    acc[0] += wgt * x0.x; acc[1] += wgt * x0.y; acc[2] += wgt * x0.z; acc[3] += wgt * x0.w;
    acc[4] += wgt * x1.x; acc[5] += wgt * x1.y; acc[6] += wgt * x1.z; acc[7] += wgt * x1.w;
  }
  const float inv = s_inv[i];
  const int t = m / a.G, g = m % a.G, hq = hk * a.G + g;
  uint32_t packed[4];
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    float y0 = acc[j] * inv, y1 = acc[j + 1] * inv;
    if (a.gate) {
      const uint16_t* gp = a.gate + ((int64_t)b * a.T + t) * a.gate_st + (int64_t)hq * a.gate_hs + c + j;
      // the attention output is rounded to bf16 before the gate, as the torch path does
      y0 = bf2f(f2bf(y0)) * (1.f / (1.f + __expf(-bf2f(gp[0]))));
      y1 = bf2f(f2bf(y1)) * (1.f / (1.f + __expf(-bf2f(gp[1]))));
    }
    packed[j / 2] = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
  }
  *reinterpret_cast<u32x4*>(a.out + (((int64_t)b * a.T + t) * a.Hq + hq) * a.D + c) =
      u32x4{packed[0], packed[1], packed[2], packed[3]};
}

// Splits per (sequence, KV head, query tile): enough workgroups to cover the CUs (~512 in all), but
// at least 4 key blocks per split so one split's O partial (rows x D fp32) stays small next to the
// keys it reads.
int64_t plan_splits(int64_t B, int64_t Hkv, int64_t QT, int64_t max_keys, int64_t splits) {
  if (splits > 0) return splits;
  const int64_t nblk = cdiv(max_keys, kKB);
  int64_t s = cdiv(512, B * Hkv * QT);
  const int64_t by_len = cdiv(nblk, 4);
  if (s > by_len) s = by_len;
  if (s > kMaxSplits) s = kMaxSplits;
  return s < 1 ? 1 : s;
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_attn_canvas_scratch_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                                   int64_t max_keys, int64_t splits) {
  if (B <= 0 || T <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0) return 0;
  const int64_t QT = cdiv(T * (Hq / Hkv), kMT);
  const int64_t S = plan_splits(B, Hkv, QT, max_keys, splits);
  const int64_t slots = B * Hkv * QT * S;
  return align_up(slots * kMT * D * 4, 256) + 2 * align_up(slots * kMT * 4, 256);
}

extern "C" int trida_attn_canvas(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                 const int32_t* prefix_len, const uint16_t* gate, int64_t gate_row_stride,
                                 int64_t gate_head_stride, uint16_t* out, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                 int64_t Lmax, int mask_mode, int64_t n_clean, float scale, int64_t max_keys,
                                 int64_t splits, void* scratch, int64_t scratch_bytes, void* stream) {
  TRIDA_CHECK(q && k_cache && v_cache && prefix_len && out && scratch, TRIDA_ERR_NULL,
              "attn_canvas: q, k_cache, v_cache, prefix_len, out and scratch are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Lmax >= T, TRIDA_ERR_ARG,
              "attn_canvas: bad sizes B=%lld T=%lld Hq=%lld Hkv=%lld Lmax=%lld", (long long)B, (long long)T,
              (long long)Hq, (long long)Hkv, (long long)Lmax);
  TRIDA_CHECK(D == 64 || D == 128 || D == 256, TRIDA_ERR_ARG, "attn_canvas: head dim must be 64, 128 or 256");
  TRIDA_CHECK(mask_mode >= 0 && mask_mode <= 2, TRIDA_ERR_ARG, "attn_canvas: mask_mode is 0, 1 or 2");
  TRIDA_CHECK(((((uintptr_t)q) | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) == 0,
              TRIDA_ERR_ALIGN, "attn_canvas: q, caches and out must be 16-byte aligned");
  TRIDA_CHECK(gate == nullptr || (gate_head_stride >= D && gate_row_stride >= Hq * gate_head_stride - (gate_head_stride - D)),
              TRIDA_ERR_ARG, "attn_canvas: gate strides");
  const int64_t G = Hq / Hkv;
  const int64_t QT = cdiv(T * G, kMT);
  const int64_t S = plan_splits(B, Hkv, QT, max_keys > 0 ? max_keys : Lmax, splits);
  TRIDA_CHECK(S >= 1 && S <= kMaxSplits, TRIDA_ERR_ARG, "attn_canvas: 1..%d key splits", kMaxSplits);
  const int64_t need = trida_attn_canvas_scratch_bytes(B, T, Hq, Hkv, D, max_keys > 0 ? max_keys : Lmax, S);
  TRIDA_CHECK(scratch_bytes >= need, TRIDA_ERR_WORKSPACE, "attn_canvas: scratch %lld < %lld bytes",
              (long long)scratch_bytes, (long long)need);
  const int64_t slots = B * Hkv * QT * S;
  TRIDA_CHECK(slots < INT32_MAX && B * Hkv < 65535, TRIDA_ERR_ARG, "attn_canvas: grid too large");
  char* ws = static_cast<char*>(scratch);
  float* opart = reinterpret_cast<float*>(ws);
  float* mpart = reinterpret_cast<float*>(ws + align_up(slots * kMT * D * 4, 256));
  float* lpart = reinterpret_cast<float*>(ws + align_up(slots * kMT * D * 4, 256) + align_up(slots * kMT * 4, 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  AttnArgs a{q, k_cache, v_cache, prefix_len, opart, mpart, lpart, (int)T, (int)Hq, (int)Hkv, (int)G,
             (int)Lmax, (int)S, (int)QT, mask_mode, (int)n_clean, scale * kLog2e};
  const dim3 grid((unsigned)slots);
  switch (D) {
    case 64: hipLaunchKernelGGL(attn_partial_kernel<64>, grid, dim3(kNW * kWave), 0, st, a); break;
    case 128: hipLaunchKernelGGL(attn_partial_kernel<128>, grid, dim3(kNW * kWave), 0, st, a); break;
    default: hipLaunchKernelGGL(attn_partial_kernel<256>, grid, dim3(kNW * kWave), 0, st, a); break;
  }
  int rc = launch_status("attn_canvas/partial");
  if (rc) return rc;
  CombineArgs c{opart, mpart, lpart, gate, out, (int)T, (int)Hq, (int)Hkv, (int)G, (int)D, (int)S, (int)QT,
                gate_row_stride, gate_head_stride};
  const int64_t rows_per_block = 256 / (D / 8);
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)cdiv(T * G, rows_per_block), (unsigned)(B * Hkv)), dim3(256),
                     0, st, c);
  return launch_status("attn_canvas/combine");
}
