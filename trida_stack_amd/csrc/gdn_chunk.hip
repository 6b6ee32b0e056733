// Gated delta rule, chunked WY / UT form on MFMA (gfx950), with the block-causal canvas readout and the
// rollback to an accepted prefix of the block.
//
// Per value head, one chunk of C = 16 * NB rows with cumulative log decay G_t = sum_{s<=t} g_s inside the
// chunk and St = S^T [Dk, Dv] at the chunk start (S as stored: [Dv, Dk], row v = column v of St):
//   A[t][s]   = beta_t (k_t . k_s) e^{G_t - G_s}   (s < t)        T = (I + A)^{-1}
//   Aqk[t][s] = (q_t . k_s) e^{G_t - G_s}           (s <= t)
//   v_new     = T diag(beta) (V - e^{G} (K St))     the delta of every row against the chunk-start state
//   o         = scale (e^{G} (Q St) + Aqk v_new)
//   St'       = e^{G_{n-1}} St + K^T diag(e^{G_{n-1} - G}) v_new[:n]    (the first n rows absorbed)
// the chunk-parallel form of S = e^g S; S += beta (v - S k) k^T; o = S q. Every exponent is <= 0, so
// nothing overflows under strong decay.
//
// T is inverted in 16 x 16 blocks: D_i = (I + A_ii)^{-1} by forward substitution (one lane per column),
// N_ik = D_i A_ik, then block rows T_ij = -sum_{k=j}^{i-1} N_ik T_kj (T_ii = D_i).
//
// Precision: products that feed the state (K St, T diag(beta) R, K^T v', and the inverse) split their
// fp32 operands into bf16 hi + lo parts and sum hi*hi + hi*lo + lo*hi on v_mfma_f32_16x16x32_bf16 /
// 16x16x16 (about 16 mantissa bits, fp32 accumulation); products that only feed the bf16 output (Q St,
// Aqk v_new) use the hi parts. Keys, queries and values are bf16 inputs and enter exactly.
//
// MFMA lane layouts (wave64): 16x16x32 A fragment = row (l % 16), k = 8 (l / 16) .. + 7; B fragment =
// column (l % 16), same k; 16x16x16 uses k = 4 (l / 16) .. + 3; the accumulator holds rows
// 4 (l / 16) .. + 3 of column (l % 16).
//
// Kernels:
//   gdr_chunk_prep   (sequence, chunk of 64 rows, value head): T diag(beta) (hi / lo) and Aqk (hi) of the
//                    chunk into a workspace, in the swizzled LDS layout the scan copies back verbatim.
//   gdr_chunk_scan   (sequence, value head, Dv slice): the chunks in order; the state slice stays in MFMA
//                    accumulators from the first chunk to the last.
//   gdr_chunk_fused  (sequence, value head, Dv slice): one chunk of T <= 64 rows (a canvas block) with
//                    prep and scan in one launch; causal_mode 2 rows read the block-end state; without
//                    an output it is the rollback (state after n_keep rows).
#include <math.h>

#include "common.h"
#include "gdn_block.h"
#include "gdn_prefix.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kNT = 256;  // 4 waves
constexpr int kNW = kNT / kWave;
constexpr int kChunk = 64;  // rows per chunk of the multi-chunk path

__device__ __forceinline__ f32x4 mfma32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void split(float x, uint16_t& hi, uint16_t& lo) {
  hi = f2bf(x);
  lo = f2bf(x - bf2f(hi));
}
__device__ __forceinline__ void split4(const float* x, s16x4& hi, s16x4& lo) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    uint16_t h, l;
    split(x[r], h, l);
    hi[r] = (short)h;
    lo[r] = (short)l;
  }
}
// hi*hi + hi*lo + lo*hi of two fp32 16x16 blocks given as 4-element fragments
__device__ __forceinline__ f32x4 mm3(const float* a, const float* b, f32x4 c) {
  s16x4 ah, al, bh, bl;
  split4(a, ah, al);
  split4(b, bh, bl);
  c = mfma16(ah, bh, c);
  c = mfma16(ah, bl, c);
  return mfma16(al, bh, c);
}

// bf16 matrix [rows][COLS] in LDS, 16-byte groups XOR-swizzled by the row so that the 8-element fragment
// reads of 16 consecutive rows (and the 4-element writes from accumulator layouts) spread over banks.
template <int COLS>
__device__ __forceinline__ int sw(int r, int c) {
  constexpr int G = COLS / 8;
  constexpr int M = (G >= 8 ? 8 : G) - 1;
  return r * COLS + ((((c >> 3) ^ (r & M))) << 3) + (c & 7);
}
template <int COLS>
__device__ __forceinline__ u32x4 frag8(const uint16_t* m, int r, int c) {
  return *reinterpret_cast<const u32x4*>(&m[sw<COLS>(r, c)]);
}
// 4 bf16 (hi or lo of 4 fp32 values) at row r, columns c .. c + 3 (c % 4 == 0)
template <int COLS>
__device__ __forceinline__ void put4(uint16_t* m, int r, int c, const uint16_t* v) {
  u32x2 w;
  w.x = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
  w.y = (uint32_t)v[2] | ((uint32_t)v[3] << 16);
  *reinterpret_cast<u32x2*>(&m[sw<COLS>(r, c)]) = w;
}
template <int COLS>
__device__ __forceinline__ void put4_split(uint16_t* mh, uint16_t* ml, int r, int c, const float* x) {
  uint16_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split(x[i], h[i], l[i]);
  put4<COLS>(mh, r, c, h);
  if (ml) put4<COLS>(ml, r, c, l);
}

// LDS plan of one workgroup (bytes). The prep's fp32 scratch (A then N in place, T) overlays the
// scan-only buffers, which are first written after the prep is done.
template <int DK, int NB, int DVS>
struct Lay {
  static constexpr int C = 16 * NB;
  static constexpr int PS = C + 4;  // fp32 row stride of the prep matrices
  static constexpr int kK = 0;                         // K   [C][DK]  bf16 (A operand, rows = t)
  static constexpr int kKt = kK + C * DK * 2;          // K^T [DK][C]  bf16 (A operand, rows = dk)
  static constexpr int kQ = kKt + DK * C * 2;          // Q   [C][DK]  bf16
  static constexpr int kV = kQ + C * DK * 2;           // V   [C][DVS] fp32 (this workgroup's columns)
  static constexpr int kG = kV + C * DVS * 4;          // G   [C] fp32 (cumulative log decay)
  static constexpr int kBeta = kG + C * 4;             // beta [C] fp32
  static constexpr int kTbH = kBeta + C * 4;           // T diag(beta) [C][C] bf16 hi / lo
  static constexpr int kTbL = kTbH + C * C * 2;
  static constexpr int kAq = kTbL + C * C * 2;         // Aqk [C][C] bf16 hi
  static constexpr int kSH = kAq + C * C * 2;          // St slice as [DVS][DK] bf16 hi / lo (B operand)
  static constexpr int kSL = kSH + DVS * DK * 2;
  static constexpr int kRH = kSL + DVS * DK * 2;       // R, v_new, v' as [DVS][C] bf16 (B operands)
  static constexpr int kRL = kRH + DVS * C * 2;
  static constexpr int kVn = kRL + DVS * C * 2;
  static constexpr int kVpH = kVn + DVS * C * 2;
  static constexpr int kVpL = kVpH + DVS * C * 2;
  static constexpr int kEnd = kVpL + DVS * C * 2;
  static constexpr int kPA = kSH;                      // prep: A, then N in place   [C][PS] fp32
  static constexpr int kPT = kPA + C * PS * 4;         // prep: T                    [C][PS] fp32
  static constexpr int kPEnd = kPT + C * PS * 4;
  static constexpr int BYTES = kPEnd > kEnd ? kPEnd : kEnd;
  static_assert(BYTES <= 160 * 1024, "LDS plan exceeds 160 KiB");
};

struct ChunkArgs {
  const uint16_t* q;       // [B, T, Hk, DK]
  const uint16_t* k;       // [B, T, Hk, DK]
  const uint16_t* v;       // [B, T, Hv, Dv]
  const float* g;          // [B, T, Hv]
  const float* beta;       // [B, T, Hv]
  const float* state_in;   // [B, Hv, Dv, DK]
  uint16_t* out;           // [B, T, Hv, Dv] or null (no readout)
  float* state_out;        // [B, Hv, Dv, DK] or null
  const int32_t* n_keep;   // [seq_mod] or null: rows absorbed into state_out
  uint16_t* ws;            // prep workspace: [B, nchunks, Hv][3][64 x 64] bf16
  int T, Hk, Hv, Dv, nc, seq_mod, nchunks;
  float scale;
  const int32_t* cu;       // [B + 1] packed ragged rows, or null (B x T rows)
  const int32_t* sidx;     // [B] state_in / state_out row of sequence b, or null (row b)
};

// Rows of sequence b: [row0, row0 + n) of the packed arrays (n <= T).
struct SeqRows {
  int64_t row0;
  int n;
};
__device__ __forceinline__ SeqRows seq_rows(const ChunkArgs& a, int b) {
  if (!a.cu) return {(int64_t)b * a.T, a.T};
  const int lo = a.cu[b];
  return {lo, max(0, min(a.cu[b + 1] - lo, a.T))};
}
__device__ __forceinline__ int64_t state_row(const ChunkArgs& a, int b) { return a.sidx ? a.sidx[b] : b; }

// ---------------------------------------------------------------------------------------------- staging
// Workspace block of one (sequence, chunk, value head): T diag(beta) hi, lo and Aqk hi, 64 x 64 bf16 each.
constexpr int kWsElems = 3 * kChunk * kChunk;
static_assert(kWsElems * 2 >= kPrefixWsBytes, "the workspace also serves the prefix kernels");

// Rows [t0, t0 + cc) of one chunk (rows cc..C-1 read as zero), staged in two steps so that every global
// load of a chunk is in flight at once: load() issues them into registers, store() writes LDS (K
// row-major and transposed, Q, the V slice as fp32, G = inclusive cumsum of g, beta and, with WS, the
// chunk's prep block from the workspace). The multi-chunk scan loads chunk c + 1 while computing c.
template <int DK, int NB, int DVS, bool WANT_Q, bool WANT_V, bool WS>
struct Stage {
  using L = Lay<DK, NB, DVS>;
  static constexpr int C = L::C;
  static constexpr int KSQ = (C / 8) * (DK / 8);  // 8 x 8 squares of K (rows t, columns dk)
  static constexpr int KSQ_PT = (KSQ + kNT - 1) / kNT;
  static constexpr int QP = C * DK / 8;           // 16-byte pieces of Q
  static constexpr int QP_PT = WANT_Q ? (QP + kNT - 1) / kNT : 0;
  static constexpr int VP = C * DVS / 8;          // 16-byte pieces of the V slice
  static constexpr int VP_PT = WANT_V ? (VP + kNT - 1) / kNT : 0;
  static constexpr int WP = kWsElems / 8;
  static constexpr int WP_PT = WS ? (WP + kNT - 1) / kNT : 0;
  u32x4 k[KSQ_PT][8];
  u32x4 q[QP_PT > 0 ? QP_PT : 1];
  u32x4 v[VP_PT > 0 ? VP_PT : 1];
  u32x4 ws[WP_PT > 0 ? WP_PT : 1];
  float g, beta;

  // b: the sequence (workspace block); r0: its first row in the packed arrays
  __device__ __forceinline__ void load(const ChunkArgs& a, int b, int64_t r0, int h, int hk, int dv0, int t0,
                                       int cc, int chunk) {
    const int tid = threadIdx.x;
    const int64_t qk_row = (int64_t)a.Hk * DK;
    const uint16_t* kb = a.k + (r0 + t0) * qk_row + (int64_t)hk * DK;
#pragma unroll
    for (int i = 0; i < KSQ_PT; ++i) {
      const int sq = tid + i * kNT;
      const int rb = sq / (DK / 8), cb = sq % (DK / 8);
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const int t = rb * 8 + r;
        k[i][r] = (sq < KSQ && t < cc) ? *reinterpret_cast<const u32x4*>(kb + (int64_t)t * qk_row + cb * 8)
                                       : u32x4{0, 0, 0, 0};
      }
    }
    if (WANT_Q) {
      const uint16_t* qb = a.q + (r0 + t0) * qk_row + (int64_t)hk * DK;
#pragma unroll
      for (int i = 0; i < QP_PT; ++i) {
        const int p = tid + i * kNT;
        const int t = p / (DK / 8), c = (p % (DK / 8)) * 8;
        q[i] = (p < QP && t < cc) ? *reinterpret_cast<const u32x4*>(qb + (int64_t)t * qk_row + c)
                                  : u32x4{0, 0, 0, 0};
      }
    }
    if (WANT_V) {
      const int64_t v_row = (int64_t)a.Hv * a.Dv;
      const uint16_t* vb = a.v + (r0 + t0) * v_row + (int64_t)h * a.Dv + dv0;
#pragma unroll
      for (int i = 0; i < VP_PT; ++i) {
        const int p = tid + i * kNT;
        const int t = p / (DVS / 8), c = (p % (DVS / 8)) * 8;
        v[i] = (p < VP && t < cc) ? *reinterpret_cast<const u32x4*>(vb + (int64_t)t * v_row + c)
                                  : u32x4{0, 0, 0, 0};
      }
    }
    if (WS) {
      const u32x4* src =
          reinterpret_cast<const u32x4*>(a.ws + (((int64_t)b * a.nchunks + chunk) * a.Hv + h) * kWsElems);
#pragma unroll
      for (int i = 0; i < WP_PT; ++i) {
        const int p = tid + i * kNT;
        ws[i] = p < WP ? src[p] : u32x4{0, 0, 0, 0};
      }
    }
    if (tid < kWave) {
      const int64_t gi = (r0 + t0 + tid) * a.Hv + h;
      const bool in = tid < cc && tid < C;
      g = in ? a.g[gi] : 0.f;
      beta = in ? a.beta[gi] : 0.f;
    }
  }

  __device__ __forceinline__ void store(unsigned char* smem) {
    uint16_t* sK = reinterpret_cast<uint16_t*>(smem + L::kK);
    uint16_t* sKt = reinterpret_cast<uint16_t*>(smem + L::kKt);
    uint16_t* sQ = reinterpret_cast<uint16_t*>(smem + L::kQ);
    float* sV = reinterpret_cast<float*>(smem + L::kV);
    float* sG = reinterpret_cast<float*>(smem + L::kG);
    float* sBeta = reinterpret_cast<float*>(smem + L::kBeta);
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < KSQ_PT; ++i) {
      const int sq = tid + i * kNT;
      if (sq >= KSQ) continue;
      const int rb = sq / (DK / 8), cb = sq % (DK / 8);
#pragma unroll
      for (int r = 0; r < 8; ++r) *reinterpret_cast<u32x4*>(&sK[sw<DK>(rb * 8 + r, cb * 8)]) = k[i][r];
#pragma unroll
      for (int j = 0; j < 8; ++j) {  // column dk = cb * 8 + j of the 8 rows
        uint16_t e[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const uint32_t w = k[i][r][j >> 1];
          e[r] = (uint16_t)((j & 1) ? (w >> 16) : (w & 0xffffu));
        }
        u32x4 o;
        o.x = (uint32_t)e[0] | ((uint32_t)e[1] << 16);
        o.y = (uint32_t)e[2] | ((uint32_t)e[3] << 16);
        o.z = (uint32_t)e[4] | ((uint32_t)e[5] << 16);
        o.w = (uint32_t)e[6] | ((uint32_t)e[7] << 16);
        *reinterpret_cast<u32x4*>(&sKt[sw<C>(cb * 8 + j, rb * 8)]) = o;
      }
    }
    if (WANT_Q) {
#pragma unroll
      for (int i = 0; i < QP_PT; ++i) {
        const int p = tid + i * kNT;
        if (p < QP) *reinterpret_cast<u32x4*>(&sQ[sw<DK>(p / (DK / 8), (p % (DK / 8)) * 8)]) = q[i];
      }
    }
    if (WANT_V) {
#pragma unroll
      for (int i = 0; i < VP_PT; ++i) {
        const int p = tid + i * kNT;
        if (p >= VP) continue;
        const int t = p / (DVS / 8), c = (p % (DVS / 8)) * 8;
        f32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          lo[2 * e] = bf2f((uint16_t)(v[i][e] & 0xffffu));
          lo[2 * e + 1] = bf2f((uint16_t)(v[i][e] >> 16));
          hi[2 * e] = bf2f((uint16_t)(v[i][2 + e] & 0xffffu));
          hi[2 * e + 1] = bf2f((uint16_t)(v[i][2 + e] >> 16));
        }
        *reinterpret_cast<f32x4*>(&sV[t * DVS + c]) = lo;
        *reinterpret_cast<f32x4*>(&sV[t * DVS + c + 4]) = hi;
      }
    }
    if (WS) {
      u32x4* dst = reinterpret_cast<u32x4*>(smem + L::kTbH);  // TbH, TbL, Aq are contiguous
#pragma unroll
      for (int i = 0; i < WP_PT; ++i) {
        const int p = tid + i * kNT;
        if (p < WP) dst[p] = ws[i];
      }
    }
    if (tid < kWave) {  // G = inclusive cumsum of g over the chunk (rows past cc carry the last value)
      float gv = g;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float o = __shfl_up(gv, off, kWave);
        if (tid >= off) gv += o;
      }
      if (tid < C) {
        sG[tid] = gv;
        sBeta[tid] = beta;
      }
    }
  }
};

// ---------------------------------------------------------------------------------------------- prep
// From sK, sQ, sG, sBeta: T diag(beta) (hi / lo) into sTbH / sTbL and Aqk (hi) into sAq (when WANT_Q).
// Uses and ends with __syncthreads; the caller synchronises after staging.
template <int DK, int NB, int DVS, bool WANT_Q>
__device__ void prep_chunk(unsigned char* smem) {
  using L = Lay<DK, NB, DVS>;
  constexpr int C = L::C, PS = L::PS;
  const uint16_t* sK = reinterpret_cast<const uint16_t*>(smem + L::kK);
  const uint16_t* sQ = reinterpret_cast<const uint16_t*>(smem + L::kQ);
  const float* sG = reinterpret_cast<const float*>(smem + L::kG);
  const float* sBeta = reinterpret_cast<const float*>(smem + L::kBeta);
  uint16_t* sTbH = reinterpret_cast<uint16_t*>(smem + L::kTbH);
  uint16_t* sTbL = reinterpret_cast<uint16_t*>(smem + L::kTbL);
  uint16_t* sAq = reinterpret_cast<uint16_t*>(smem + L::kAq);
  float* pA = reinterpret_cast<float*>(smem + L::kPA);
  float* pT = reinterpret_cast<float*>(smem + L::kPT);
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int lr = l % 16, lg = l / 16;

  // zero T diag(beta) and Aqk (their upper blocks stay zero)
  for (int p = tid; p < C * C / 8; p += kNT) {
    reinterpret_cast<u32x4*>(sTbH)[p] = u32x4{0, 0, 0, 0};
    reinterpret_cast<u32x4*>(sTbL)[p] = u32x4{0, 0, 0, 0};
    if (WANT_Q) reinterpret_cast<u32x4*>(sAq)[p] = u32x4{0, 0, 0, 0};
  }
  __syncthreads();
  // P1: K K^T and Q K^T on the lower block tiles (i >= j)
  constexpr int NTL = NB * (NB + 1) / 2;
  for (int tile = w; tile < NTL; tile += kNW) {
    int i = 0, rem = tile;
    while (rem > i) {
      rem -= i + 1;
      ++i;
    }
    const int j = rem;
    f32x4 kk = {0.f, 0.f, 0.f, 0.f}, qk = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < DK / 32; ++kc) {
      const u32x4 bf = frag8<DK>(sK, 16 * j + lr, 32 * kc + 8 * lg);
      kk = mfma32(frag8<DK>(sK, 16 * i + lr, 32 * kc + 8 * lg), bf, kk);
      if (WANT_Q) qk = mfma32(frag8<DK>(sQ, 16 * i + lr, 32 * kc + 8 * lg), bf, qk);
    }
    const int s = 16 * j + lr;
    const float gs = sG[s];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = 16 * i + 4 * lg + r;
      const float dec = __expf(sG[t] - gs);
      pA[t * PS + s] = s < t ? sBeta[t] * kk[r] * dec : 0.f;
      if (WANT_Q) sAq[sw<C>(t, s)] = f2bf(s <= t ? qk[r] * dec : 0.f);
    }
  }
  __syncthreads();
  // P2: diagonal blocks D_i = (I + A_ii)^{-1}, one lane per column (wave 0, block = lane / 16)
  if (w == 0 && lg < NB) {
    const int o = 16 * lg;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float s = (i == lr) ? 1.f : 0.f;
      const float* arow = pA + (o + i) * PS + o;
#pragma unroll
      for (int j = 0; j < i; ++j) s = fmaf(-arow[j], x[j], s);
      x[i] = s;
    }
    const float bs = sBeta[o + lr];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      pT[(o + i) * PS + o + lr] = x[i];
      uint16_t hi, lo;
      split(x[i] * bs, hi, lo);
      sTbH[sw<C>(o + i, o + lr)] = hi;
      sTbL[sw<C>(o + i, o + lr)] = lo;
    }
  }
  if (NB == 1) {
    __syncthreads();
    return;
  }
  __syncthreads();
  // P3: N_ik = D_i A_ik (i > k), in place over A_ik
  constexpr int NOFF = NB * (NB - 1) / 2;
  for (int tile = w; tile < NOFF; tile += kNW) {
    int i = 1, rem = tile;
    while (rem >= i) {
      rem -= i;
      ++i;
    }
    const int kb = rem;
    float af[4], bfv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      af[r] = pT[(16 * i + lr) * PS + 16 * i + 4 * lg + r];     // D_i [row lr][k]
      bfv[r] = pA[(16 * i + 4 * lg + r) * PS + 16 * kb + lr];   // A_ik [k][col lr]
    }
    const f32x4 n = mm3(af, bfv, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
    for (int r = 0; r < 4; ++r) pA[(16 * i + 4 * lg + r) * PS + 16 * kb + lr] = n[r];
  }
  // P4: block rows T_ij = -sum_{k=j}^{i-1} N_ik T_kj
#pragma unroll
  for (int i = 1; i < NB; ++i) {
    __syncthreads();
    if (w < i) {
      const int j = w;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int kb = j; kb < i; ++kb) {
        float af[4], bfv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          af[r] = pA[(16 * i + lr) * PS + 16 * kb + 4 * lg + r];   // N_ik [row lr][k]
          bfv[r] = pT[(16 * kb + 4 * lg + r) * PS + 16 * j + lr];  // T_kj [k][col lr]
        }
        acc = mm3(af, bfv, acc);
      }
      const int s = 16 * j + lr;
      const float bs = sBeta[s];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * i + 4 * lg + r;
        const float tv = -acc[r];
        pT[t * PS + s] = tv;
        uint16_t hi, lo;
        split(tv * bs, hi, lo);
        sTbH[sw<C>(t, s)] = hi;
        sTbL[sw<C>(t, s)] = lo;
      }
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------- scan
// State slice registers: wave w owns the dk row tiles w, w + 4, ... (< DK / 16) and every dv column tile.
template <int DK>
struct StTiles {
  static constexpr int NMT = DK / 16;
  static constexpr int PER = (NMT + kNW - 1) / kNW;
};

template <int DK, int DVS>
__device__ __forceinline__ void load_state(f32x4 (&st)[StTiles<DK>::PER][DVS / 16], const float* sp, int w, int l) {
#pragma unroll
  for (int m = 0; m < StTiles<DK>::PER; ++m) {
    const int mt = w + kNW * m;
#pragma unroll
    for (int ct = 0; ct < DVS / 16; ++ct) {
      if (mt < StTiles<DK>::NMT)
        st[m][ct] = *reinterpret_cast<const f32x4*>(sp + (int64_t)(16 * ct + l % 16) * DK + 16 * mt + 4 * (l / 16));
      else
        st[m][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
}
template <int DK, int DVS>
__device__ __forceinline__ void store_state(const f32x4 (&st)[StTiles<DK>::PER][DVS / 16], float* sp, int w, int l) {
#pragma unroll
  for (int m = 0; m < StTiles<DK>::PER; ++m) {
    const int mt = w + kNW * m;
    if (mt >= StTiles<DK>::NMT) continue;
#pragma unroll
    for (int ct = 0; ct < DVS / 16; ++ct)
      *reinterpret_cast<f32x4*>(sp + (int64_t)(16 * ct + l % 16) * DK + 16 * mt + 4 * (l / 16)) = st[m][ct];
  }
}
// St (hi / lo) into sSH / sSL as [dv][dk]
template <int DK, int NB, int DVS>
__device__ __forceinline__ void put_state(unsigned char* smem, const f32x4 (&st)[StTiles<DK>::PER][DVS / 16], int w,
                                          int l) {
  using L = Lay<DK, NB, DVS>;
  uint16_t* sSH = reinterpret_cast<uint16_t*>(smem + L::kSH);
  uint16_t* sSL = reinterpret_cast<uint16_t*>(smem + L::kSL);
#pragma unroll
  for (int m = 0; m < StTiles<DK>::PER; ++m) {
    const int mt = w + kNW * m;
    if (mt >= StTiles<DK>::NMT) continue;
#pragma unroll
    for (int ct = 0; ct < DVS / 16; ++ct) {
      float x[4] = {st[m][ct][0], st[m][ct][1], st[m][ct][2], st[m][ct][3]};
      put4_split<DK>(sSH, sSL, 16 * ct + l % 16, 16 * mt + 4 * (l / 16), x);
    }
  }
}

// One chunk (LDS staged and prepped): rows t < cc; the first n_abs rows are absorbed into the state;
// rows t < n_out get the chunk readout written to out_rows (row t at out_rows + t * out_stride), when
// out_rows is not null. Ends with the state updated in registers.
template <int DK, int NB, int DVS>
__device__ void scan_chunk(unsigned char* smem, f32x4 (&st)[StTiles<DK>::PER][DVS / 16], int cc, int n_abs,
                           int n_out, uint16_t* out_rows, int64_t out_stride, float scale) {
  using L = Lay<DK, NB, DVS>;
  constexpr int C = L::C, NCT = DVS / 16;
  const uint16_t* sK = reinterpret_cast<const uint16_t*>(smem + L::kK);
  const uint16_t* sKt = reinterpret_cast<const uint16_t*>(smem + L::kKt);
  const uint16_t* sQ = reinterpret_cast<const uint16_t*>(smem + L::kQ);
  const float* sV = reinterpret_cast<const float*>(smem + L::kV);
  const float* sG = reinterpret_cast<const float*>(smem + L::kG);
  const uint16_t* sTbH = reinterpret_cast<const uint16_t*>(smem + L::kTbH);
  const uint16_t* sTbL = reinterpret_cast<const uint16_t*>(smem + L::kTbL);
  const uint16_t* sAq = reinterpret_cast<const uint16_t*>(smem + L::kAq);
  uint16_t* sSH = reinterpret_cast<uint16_t*>(smem + L::kSH);
  uint16_t* sSL = reinterpret_cast<uint16_t*>(smem + L::kSL);
  uint16_t* sRH = reinterpret_cast<uint16_t*>(smem + L::kRH);
  uint16_t* sRL = reinterpret_cast<uint16_t*>(smem + L::kRL);
  uint16_t* sVn = reinterpret_cast<uint16_t*>(smem + L::kVn);
  uint16_t* sVpH = reinterpret_cast<uint16_t*>(smem + L::kVpH);
  uint16_t* sVpL = reinterpret_cast<uint16_t*>(smem + L::kVpL);
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int lr = l % 16, lg = l / 16;
  const bool want_out = out_rows != nullptr && n_out > 0;
  const bool row_wave = w < NB;  // wave w owns chunk rows [16 w, 16 w + 16)

  put_state<DK, NB, DVS>(smem, st, w, l);
  __syncthreads();
  // K St (hi + lo) and Q St (hi); R = V - e^G K St
  f32x4 qs[NCT];
  if (row_wave) {
    f32x4 ks[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) ks[ct] = qs[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < DK / 32; ++kc) {
      const u32x4 af = frag8<DK>(sK, 16 * w + lr, 32 * kc + 8 * lg);
      u32x4 qf;
      if (want_out) qf = frag8<DK>(sQ, 16 * w + lr, 32 * kc + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const u32x4 sh = frag8<DK>(sSH, 16 * ct + lr, 32 * kc + 8 * lg);
        const u32x4 sl = frag8<DK>(sSL, 16 * ct + lr, 32 * kc + 8 * lg);
        ks[ct] = mfma32(af, sh, ks[ct]);
        ks[ct] = mfma32(af, sl, ks[ct]);
        if (want_out) qs[ct] = mfma32(qf, sh, qs[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      float r[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * lg + i;
        const float eg = __expf(sG[t]);
        r[i] = sV[t * DVS + 16 * ct + lr] - eg * ks[ct][i];
        qs[ct][i] *= eg;
      }
      put4_split<C>(sRH, sRL, 16 * ct + lr, 16 * w + 4 * lg, r);
    }
  }
  __syncthreads();
  // v_new = T diag(beta) R (hi*hi + hi*lo + lo*hi); v' = e^{G_{n-1} - G} v_new on the absorbed rows
  const float gl = n_abs > 0 ? sG[n_abs - 1] : 0.f;
  if (row_wave) {
    f32x4 vn[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) vn[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < C / 32; ++kc) {
      if (32 * kc > 16 * w + 15) break;  // T is lower triangular
      const u32x4 th = frag8<C>(sTbH, 16 * w + lr, 32 * kc + 8 * lg);
      const u32x4 tl = frag8<C>(sTbL, 16 * w + lr, 32 * kc + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const u32x4 rh = frag8<C>(sRH, 16 * ct + lr, 32 * kc + 8 * lg);
        const u32x4 rl = frag8<C>(sRL, 16 * ct + lr, 32 * kc + 8 * lg);
        vn[ct] = mfma32(th, rh, vn[ct]);
        vn[ct] = mfma32(th, rl, vn[ct]);
        vn[ct] = mfma32(tl, rh, vn[ct]);
      }
    }
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      float x[4], vp[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * w + 4 * lg + i;
        x[i] = vn[ct][i];
        vp[i] = t < n_abs ? __expf(gl - sG[t]) * vn[ct][i] : 0.f;
      }
      if (want_out) put4_split<C>(sVn, nullptr, 16 * ct + lr, 16 * w + 4 * lg, x);
      put4_split<C>(sVpH, sVpL, 16 * ct + lr, 16 * w + 4 * lg, vp);
    }
  }
  __syncthreads();
  // o = scale (e^G Q St + Aqk v_new)
  if (want_out && row_wave) {
#pragma unroll
    for (int kc = 0; kc < C / 32; ++kc) {
      if (32 * kc > 16 * w + 15) break;
      const u32x4 aq = frag8<C>(sAq, 16 * w + lr, 32 * kc + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) qs[ct] = mfma32(aq, frag8<C>(sVn, 16 * ct + lr, 32 * kc + 8 * lg), qs[ct]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * lg + i;
      if (t < n_out && t < cc) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) out_rows[(int64_t)t * out_stride + 16 * ct + lr] = f2bf(scale * qs[ct][i]);
      }
    }
  }
  // St = e^{G_{n-1}} St + K^T v' (hi + lo)
  if (n_abs > 0) {
    const float dl = __expf(gl);
#pragma unroll
    for (int m = 0; m < StTiles<DK>::PER; ++m) {
      const int mt = w + kNW * m;
      if (mt >= StTiles<DK>::NMT) continue;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) st[m][ct][i] *= dl;
#pragma unroll
      for (int kc = 0; kc < C / 32; ++kc) {
        const u32x4 kt = frag8<C>(sKt, 16 * mt + lr, 32 * kc + 8 * lg);
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) {
          st[m][ct] = mfma32(kt, frag8<C>(sVpH, 16 * ct + lr, 32 * kc + 8 * lg), st[m][ct]);
          st[m][ct] = mfma32(kt, frag8<C>(sVpL, 16 * ct + lr, 32 * kc + 8 * lg), st[m][ct]);
        }
      }
    }
  }
}

// MASK rows of a canvas block: rows t in [nc, cc) read the block-end state St: o_t = scale q_t . St.
template <int DK, int NB, int DVS>
__device__ void mask_rows(unsigned char* smem, const f32x4 (&st)[StTiles<DK>::PER][DVS / 16], int nc, int cc,
                          uint16_t* out_rows, int64_t out_stride, float scale) {
  using L = Lay<DK, NB, DVS>;
  constexpr int NCT = DVS / 16;
  const uint16_t* sQ = reinterpret_cast<const uint16_t*>(smem + L::kQ);
  const uint16_t* sSH = reinterpret_cast<const uint16_t*>(smem + L::kSH);
  const uint16_t* sSL = reinterpret_cast<const uint16_t*>(smem + L::kSL);
  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int lr = l % 16, lg = l / 16;
  __syncthreads();  // every wave is done reading sSH / sSL of the scan
  put_state<DK, NB, DVS>(smem, st, w, l);
  __syncthreads();
  if (w < NB && 16 * w + 15 >= nc && 16 * w < cc) {
    f32x4 qs[NCT];
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) qs[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < DK / 32; ++kc) {
      const u32x4 qf = frag8<DK>(sQ, 16 * w + lr, 32 * kc + 8 * lg);
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        qs[ct] = mfma32(qf, frag8<DK>(sSH, 16 * ct + lr, 32 * kc + 8 * lg), qs[ct]);
        qs[ct] = mfma32(qf, frag8<DK>(sSL, 16 * ct + lr, 32 * kc + 8 * lg), qs[ct]);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = 16 * w + 4 * lg + i;
      if (t >= nc && t < cc) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) out_rows[(int64_t)t * out_stride + 16 * ct + lr] = f2bf(scale * qs[ct][i]);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------- kernels

template <int DK, bool OUT>
__global__ __launch_bounds__(kNT) void gdr_chunk_prep_kernel(ChunkArgs a) {
  using L = Lay<DK, 4, 16>;
  __shared__ __align__(16) unsigned char smem[L::BYTES];
  int idx = blockIdx.x;
  const int h = idx % a.Hv;
  idx /= a.Hv;
  const int c = idx % a.nchunks;
  const int b = idx / a.nchunks;
  const int hk = h / (a.Hv / a.Hk);
  const int t0 = c * kChunk;
  const SeqRows sr = seq_rows(a, b);
  const int cc = min(kChunk, sr.n - t0);
  if (cc <= 0) return;  // past a packed sequence's chunks (block-uniform)
  {
    Stage<DK, 4, 16, OUT, false, false> st;
    st.load(a, b, sr.row0, h, hk, 0, t0, cc, c);
    st.store(smem);
  }
  __syncthreads();
  prep_chunk<DK, 4, 16, OUT>(smem);
  u32x4* dst = reinterpret_cast<u32x4*>(a.ws + (((int64_t)b * a.nchunks + c) * a.Hv + h) * kWsElems);
  const u32x4* src = reinterpret_cast<const u32x4*>(smem + L::kTbH);  // TbH, TbL, Aq are contiguous
  for (int p = threadIdx.x; p < kWsElems / 8; p += kNT) dst[p] = src[p];
}

template <int DK, int DVS, bool OUT>
__global__ __launch_bounds__(kNT) void gdr_chunk_scan_kernel(ChunkArgs a) {
  using L = Lay<DK, 4, DVS>;
  __shared__ __align__(16) unsigned char smem[L::BYTES];
  const int slices = a.Dv / DVS;
  int idx = xcd_major(blockIdx.x, gridDim.x);  // a head's Dv slices (same chunk rows) on one XCD
  const int sl = idx % slices;
  idx /= slices;
  const int h = idx % a.Hv;
  const int b = idx / a.Hv;
  const int hk = h / (a.Hv / a.Hk);
  const int dv0 = sl * DVS;
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const SeqRows sr = seq_rows(a, b);
  const int n_tot = a.n_keep ? min(max(a.n_keep[b % a.seq_mod], 0), sr.n) : sr.n;
  // chunks to visit: all of the sequence's with a readout, else those holding absorbed rows
  const int nch = ((OUT ? sr.n : n_tot) + kChunk - 1) / kChunk;
  f32x4 st[StTiles<DK>::PER][DVS / 16];
  const int64_t soff = ((state_row(a, b) * a.Hv + h) * a.Dv + dv0) * DK;
  load_state<DK, DVS>(st, a.state_in + soff, w, l);
  const int64_t v_row = (int64_t)a.Hv * a.Dv;
  Stage<DK, 4, DVS, OUT, true, true> nx;
  if (nch > 0) nx.load(a, b, sr.row0, h, hk, dv0, 0, min(kChunk, sr.n), 0);
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * kChunk;
    const int cc = min(kChunk, sr.n - t0);
    const int n_abs = min(max(n_tot - t0, 0), cc);
    __syncthreads();  // the previous chunk's LDS reads are done
    nx.store(smem);
    __syncthreads();
    if (c + 1 < nch) nx.load(a, b, sr.row0, h, hk, dv0, t0 + kChunk, min(kChunk, sr.n - t0 - kChunk), c + 1);
    uint16_t* orow = OUT ? a.out + (sr.row0 + t0) * v_row + (int64_t)h * a.Dv + dv0 : nullptr;
    scan_chunk<DK, 4, DVS>(smem, st, cc, n_abs, cc, orow, v_row, a.scale);
  }
  if (a.state_out) store_state<DK, DVS>(st, a.state_out + soff, w, l);
}

template <int DK, int NB, int DVS, bool OUT>
__global__ __launch_bounds__(kNT) void gdr_chunk_fused_kernel(ChunkArgs a) {
  using L = Lay<DK, NB, DVS>;
  __shared__ __align__(16) unsigned char smem[L::BYTES];
  const int slices = a.Dv / DVS;
  int idx = xcd_major(blockIdx.x, gridDim.x);  // a head's Dv slices (same chunk rows) on one XCD
  const int sl = idx % slices;
  idx /= slices;
  const int h = idx % a.Hv;
  const int b = idx / a.Hv;
  const int hk = h / (a.Hv / a.Hk);
  const int dv0 = sl * DVS;
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const SeqRows sr = seq_rows(a, b);
  const int cc = sr.n;
  const int n_abs = a.n_keep ? min(max(a.n_keep[b % a.seq_mod], 0), cc) : cc;
  f32x4 st[StTiles<DK>::PER][DVS / 16];
  const int64_t soff = ((state_row(a, b) * a.Hv + h) * a.Dv + dv0) * DK;
  if (cc == 0) {  // an empty packed sequence: the state passes through
    if (a.state_out) {
      load_state<DK, DVS>(st, a.state_in + soff, w, l);
      store_state<DK, DVS>(st, a.state_out + soff, w, l);
    }
    return;
  }
  {
    Stage<DK, NB, DVS, OUT, true, false> sg;
    sg.load(a, b, sr.row0, h, hk, dv0, 0, cc, 0);
    load_state<DK, DVS>(st, a.state_in + soff, w, l);
    sg.store(smem);
  }
  __syncthreads();
  prep_chunk<DK, NB, DVS, OUT>(smem);
  const int64_t v_row = (int64_t)a.Hv * a.Dv;
  uint16_t* orow = OUT ? a.out + sr.row0 * v_row + (int64_t)h * a.Dv + dv0 : nullptr;
  const int n_out = min(a.nc, cc);
  scan_chunk<DK, NB, DVS>(smem, st, cc, n_abs, n_out, orow, v_row, a.scale);
  if (OUT && n_out < cc) mask_rows<DK, NB, DVS>(smem, st, n_out, cc, orow, v_row, a.scale);
  if (a.state_out) store_state<DK, DVS>(st, a.state_out + soff, w, l);
}

template <int DK, int NB, int DVS>
void launch_fused(const ChunkArgs& a, unsigned grid, hipStream_t stream) {
  if (a.out) hipLaunchKernelGGL((gdr_chunk_fused_kernel<DK, NB, DVS, true>), dim3(grid), dim3(kNT), 0, stream, a);
  else hipLaunchKernelGGL((gdr_chunk_fused_kernel<DK, NB, DVS, false>), dim3(grid), dim3(kNT), 0, stream, a);
}
template <int DK, int DVS>
void launch_scan(const ChunkArgs& a, unsigned grid, hipStream_t stream) {
  if (a.out) hipLaunchKernelGGL((gdr_chunk_scan_kernel<DK, DVS, true>), dim3(grid), dim3(kNT), 0, stream, a);
  else hipLaunchKernelGGL((gdr_chunk_scan_kernel<DK, DVS, false>), dim3(grid), dim3(kNT), 0, stream, a);
}

template <int DK>
int launch_dk(ChunkArgs& a, int B, hipStream_t stream) {
  const bool fused = a.T <= kChunk;
  // Dv slices: 32 columns when the grid is already wide, else 16
  const int64_t wide = (int64_t)B * a.Hv * (a.Dv / 32);
  const int dvs = (a.Dv % 32 == 0 && wide >= 512) ? 32 : 16;
  const unsigned grid = (unsigned)((int64_t)B * a.Hv * (a.Dv / dvs));
  if (fused) {
    const bool nb2 = a.T <= 32;
    if (dvs == 32) {
      if (nb2) launch_fused<DK, 2, 32>(a, grid, stream);
      else launch_fused<DK, 4, 32>(a, grid, stream);
    } else {
      if (nb2) launch_fused<DK, 2, 16>(a, grid, stream);
      else launch_fused<DK, 4, 16>(a, grid, stream);
    }
    return launch_status("gdr_chunk (single chunk)");
  }
  const unsigned pgrid = (unsigned)((int64_t)B * a.nchunks * a.Hv);
  if (a.out) hipLaunchKernelGGL((gdr_chunk_prep_kernel<DK, true>), dim3(pgrid), dim3(kNT), 0, stream, a);
  else hipLaunchKernelGGL((gdr_chunk_prep_kernel<DK, false>), dim3(pgrid), dim3(kNT), 0, stream, a);
  if (dvs == 32) launch_scan<DK, 32>(a, grid, stream);
  else launch_scan<DK, 16>(a, grid, stream);
  return launch_status("gdr_chunk (prep + scan)");
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_gdr_chunk_workspace_bytes(int64_t B, int64_t T, int64_t Hv) {
  if (B <= 0 || T <= kChunk || Hv <= 0) return 0;
  return B * cdiv(T, kChunk) * Hv * (int64_t)kWsElems * 2;
}

extern "C" int trida_gdr_chunk(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                               const float* beta, const float* state_in, uint16_t* out, float* state_out,
                               const int32_t* n_keep, int64_t seq_mod, int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                               int64_t Dk, int64_t Dv, int causal_mode, int64_t num_clean, float scale,
                               void* workspace, int64_t workspace_bytes, const int32_t* cu_seqlens,
                               const int32_t* state_idx, void* stream) {
  TRIDA_CHECK(k && v && g && beta && state_in, TRIDA_ERR_NULL, "gdr_chunk: k, v, g, beta and state_in are required");
  TRIDA_CHECK(out || state_out, TRIDA_ERR_ARG, "gdr_chunk: nothing to compute (out and state_out are both NULL)");
  TRIDA_CHECK(!out || q, TRIDA_ERR_NULL, "gdr_chunk: q is required with out");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, TRIDA_ERR_ARG,
              "gdr_chunk: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld", (long long)B, (long long)T, (long long)Hk,
              (long long)Hv);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128, TRIDA_ERR_ARG, "gdr_chunk: Dk must be 32, 64 or 128 (got %lld)",
              (long long)Dk);
  TRIDA_CHECK(Dv > 0 && Dv % 16 == 0, TRIDA_ERR_ARG, "gdr_chunk: Dv must be a multiple of 16 (got %lld)",
              (long long)Dv);
  TRIDA_CHECK(causal_mode == 1 || causal_mode == 2, TRIDA_ERR_ARG, "gdr_chunk: causal_mode is 1 or 2");
  TRIDA_CHECK(causal_mode == 1 || T <= kChunk, TRIDA_ERR_ARG,
              "gdr_chunk: causal_mode 2 (canvas readout) needs T <= %d rows", kChunk);
  TRIDA_CHECK(causal_mode == 1 || !n_keep, TRIDA_ERR_ARG, "gdr_chunk: n_keep needs causal_mode 1");
  TRIDA_CHECK(num_clean >= 0, TRIDA_ERR_ARG, "gdr_chunk: num_clean >= 0");
  TRIDA_CHECK(!n_keep || seq_mod > 0, TRIDA_ERR_ARG, "gdr_chunk: seq_mod > 0 with n_keep");
  TRIDA_CHECK(((uintptr_t)k & 15) == 0 && (!q || ((uintptr_t)q & 15) == 0) && ((uintptr_t)v & 15) == 0 &&
                  ((uintptr_t)state_in & 15) == 0 && (!state_out || ((uintptr_t)state_out & 15) == 0),
              TRIDA_ERR_ALIGN, "gdr_chunk: q, k, v and the states must be 16-byte aligned");
  TRIDA_CHECK(B * T * Hv < INT32_MAX && B * Hv * Dv < INT32_MAX, TRIDA_ERR_ARG, "gdr_chunk: problem too large");
  const int64_t nchunks = cdiv(T, kChunk);
  const int64_t need = trida_gdr_chunk_workspace_bytes(B, T, Hv);
  TRIDA_CHECK(need == 0 || (workspace && workspace_bytes >= need && ((uintptr_t)workspace & 15) == 0),
              TRIDA_ERR_WORKSPACE, "gdr_chunk: workspace of %lld bytes (16-byte aligned) required", (long long)need);
  const bool indexed = cu_seqlens || state_idx;  // the packed / state-pool forms run the kernels below
  if (!indexed && out && !state_out && !n_keep && gdr_block_supported(T, Dk, Dv)) {
    // a canvas block's readout (draft / verify / canvas passes): the single-block MFMA kernel
    BlockArgs ba{q, k, v, g, beta, state_in, out, (int)T, (int)Hk, (int)Hv, (int)Dv, causal_mode,
                 causal_mode == 2 ? (int)(num_clean < T ? num_clean : T) : (int)T, scale};
    return gdr_block_launch(ba, B, static_cast<hipStream_t>(stream));
  }
  if (!indexed && !n_keep && gdr_prefix_supported(B, T, Hv, Dk, Dv)) {
    // a prompt prefix (every row causal, the state after the last row): the chunk-parallel preparation, then
    // the scan whose chain wave holds the state
    PrefixArgs pa{q, k, v, g, beta, state_in, out, state_out, workspace, (int)T, (int)Hk, (int)Hv, (int)Dv,
                  (int)nchunks, scale};
    return gdr_prefix_launch(pa, B, static_cast<hipStream_t>(stream));
  }
  ChunkArgs a{q,        k,   v,       g,         beta,       state_in,      out,
              state_out, n_keep, static_cast<uint16_t*>(workspace), (int)T, (int)Hk, (int)Hv, (int)Dv,
              causal_mode == 2 ? (int)(num_clean < T ? num_clean : T) : (int)T, n_keep ? (int)seq_mod : 1, (int)nchunks,
              scale, cu_seqlens, state_idx};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_dk<32>(a, (int)B, st);
    case 64: return launch_dk<64>(a, (int)B, st);
    default: return launch_dk<128>(a, (int)B, st);
  }
}
