// Gated delta rule over one canvas block (T <= 64 rows, Dk = 128), the readout of a draft / verify / canvas
// pass, in the single-chunk WY / UT form on MFMA. It serves trida_gdr_chunk's readout-only blocks (out given,
// no state_out), the form the decode step runs 4-5 times per step and layer.
//
// Per (sequence, value head), with G_t = sum_{s<=t} g_s, St = S^T [Dk, Dv] the state before the block
// (S as stored [Dv, Dk]; never written) and TP = T rounded up to 16 (rows past T are zero):
//   A[t][s] = beta_t (k_t . k_s) e^{G_t - G_s} (s < t)          T = (I + A)^{-1}  (unit lower triangular)
//   R       = diag(beta) (V - diag(e^G) K St)                  v_new = T R
//   causal row t:    o_t = scale (e^{G_t} q_t St + sum_{s<=t} (q_t . k_s) e^{G_t - G_s} v_new_s)
//   block-end row t: o_t = scale (e^{G_L} q_t St + sum_{s<T} (q_t . k_s) e^{G_L - G_s} v_new_s)   (L = T - 1)
// (causal_mode 1: every row causal; 2: rows >= num_clean read the block-end state), the chunk form of
// S = e^g S; S += beta (v - S k) k^T; o = S q. Every exponent taken is <= 0.
//
// Workgroup = (sequence, value head, NWV x 32 value columns), one wave per 32 columns:
//   1. K, Q (the head's rows) and the group's V columns into LDS, the wave's St slice into registers, all
//      loads in flight together; G by a wave prefix sum;
//   2. K K^T and Q K^T (16 x 16 tiles over Dk on v_mfma_f32_16x16x32_bf16, shared out among the waves),
//      decayed and masked into A and M (the readout matrix of every row, causal or block-end);
//   3. every wave forms K St and Q St for its columns (St from HBM as split bf16 hi + lo, K and Q exact);
//      the 16 x 16 diagonal blocks T[i][i] = (I + A[i][i])^{-1} by forward substitution in fp32 (one per wave);
//   4. v_new = T R by blocks, v_new_i = T[i][i] (R_i - sum_{k<i} A[i][k] v_new_k), and
//      o = diag(e^G or e^{G_L}) Q St + M v_new on v_mfma_f32_16x16x16_bf16: the
//      accumulator layout of R and v_new (rows 4 (l / 16) + i of column l % 16) is the B operand of the
//      16x16x16 MFMA, so they never leave registers. fp32 operands enter as hi + lo bf16 with
//      hi*hi + hi*lo + lo*hi (about 16 mantissa bits; each split once); fp32 accumulation.
#include <math.h>

#include "common.h"
#include "gdn_block.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int DK = 128;
constexpr int CW = 32;  // value columns per wave

__device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
// fp32 x 4 -> bf16 hi and lo (x ~ hi + lo)
__device__ __forceinline__ void split4(f32x4 x, s16x4& hi, s16x4& lo) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const uint16_t h = f2bf(x[r]);
    hi[r] = (short)h;
    lo[r] = (short)f2bf(x[r] - bf2f(h));
  }
}
// 8 fp32 -> 8 bf16 hi and lo, packed as 16x16x32 fragments
__device__ __forceinline__ void split8(f32x4 a, f32x4 b, u32x4& hi, u32x4& lo) {
  float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t h0 = f2bf(x[2 * i]), h1 = f2bf(x[2 * i + 1]);
    h[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
    l[i] = (uint32_t)f2bf(x[2 * i] - bf2f(h0)) | ((uint32_t)f2bf(x[2 * i + 1] - bf2f(h1)) << 16);
  }
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}
// workgroup barrier that orders LDS only: waits for this wave's LDS operations, not for its global loads
// still in flight (__syncthreads' release fence would also wait for those)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// K / Q rows [TP][128] bf16 in LDS, 16-byte groups XOR-swizzled by the row (fragment reads of 16 rows
// touch distinct bank groups)
__device__ __forceinline__ int kq_off(int r, int grp) { return r * DK + ((grp ^ (r & 15)) << 3); }

template <int TP>
struct BlockLds {
  static constexpr int RT = TP / 16;
  uint16_t K[TP * DK];  // K rows; in step 4 the output tile [TP][NWV * 32] on its way out
  uint16_t Q[TP * DK];
  // 16 x 16 tiles as lane l's 16x16x16 A fragment: row l % 16, columns 4 (l / 16) .. + 4
  f32x4 A[RT * (RT + 1) / 2 * kWave];  // lower tiles (i, j <= i) of the strictly lower A, tile i (i + 1) / 2 + j
  f32x4 Tm[RT * kWave];                // the diagonal tiles of T = (I + A)^{-1}
  u32x4 M[RT * RT * kWave];            // tile (i, j) of M, {4 bf16 hi, 4 bf16 lo}
  float G[TP];
  float beta[TP];
  float rs[TP];  // the row scale of the Q St term: e^{G_t} (causal) or e^{G_L} (block-end)
};

// K K^T / Q K^T job -> 16 x 16 tile: jobs < RT (RT + 1) / 2 walk the lower triangle of K K^T row by row,
// the rest the RT x RT tiles of Q K^T
template <int RT>
__device__ __forceinline__ void job_tile(int job, int& ti, int& tj) {
  constexpr int NKK = RT * (RT + 1) / 2;
  if (job < NKK) {
    ti = 0;
#pragma unroll
    for (int x = 1; x < RT; ++x)
      if (job >= x * (x + 1) / 2) ti = x;
    tj = job - ti * (ti + 1) / 2;
  } else {
    ti = (job - NKK) / RT;
    tj = (job - NKK) % RT;
  }
}

template <int TP, int NWV>
__global__ __launch_bounds__(NWV* kWave, NWV == 4 && TP <= 48 ? 3 : 1) void gdr_block_kernel(BlockArgs a) {
  static_assert(TP % 16 == 0 && TP <= 64, "one chunk of <= 64 rows");
  constexpr int NT = NWV * kWave, RT = TP / 16;  // threads, row tiles
  __shared__ __align__(16) BlockLds<TP> sh;

  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int groups = a.Dv / (NWV * CW);
  const int grp = blockIdx.x % groups;
  const int bh = blockIdx.x / groups;
  const int b = bh / a.Hv, h = bh % a.Hv, hk = h / (a.Hv / a.Hk);
  const int T = a.T;
  const int c0 = grp * NWV * CW + w * CW;  // this wave's first value column

  // ---- 1. g and beta of row l and the K / Q rows (rows past T read row 0, in bounds, and are zeroed when
  // stored), every load issued before the first store
  float graw, braw;
  {
    const int64_t gi = ((int64_t)b * T + min(l, T - 1)) * a.Hv + h;
    graw = a.g[gi];
    braw = a.beta[gi];
    constexpr int NKQ = (TP * (DK / 8) + NT - 1) / NT;
    u32x4 kv[NKQ], qv[NKQ];
#pragma unroll
    for (int j = 0; j < NKQ; ++j) {
      const int i = min(tid + j * NT, TP * (DK / 8) - 1);
      const int t = i / (DK / 8), gi8 = i % (DK / 8);
      const int64_t row = ((int64_t)b * T + (t < T ? t : 0)) * a.Hk + hk;
      kv[j] = *reinterpret_cast<const u32x4*>(a.k + row * DK + gi8 * 8);
      qv[j] = *reinterpret_cast<const u32x4*>(a.q + row * DK + gi8 * 8);
    }
    const u32x4 z4 = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < NKQ; ++j) {
      const int i = tid + j * NT;
      if (i < TP * (DK / 8)) {
        const int t = i / (DK / 8), gi8 = i % (DK / 8);
        *reinterpret_cast<u32x4*>(&sh.K[kq_off(t, gi8)]) = t < T ? kv[j] : z4;
        *reinterpret_cast<u32x4*>(&sh.Q[kq_off(t, gi8)]) = t < T ? qv[j] : z4;
      }
    }
  }
  if (w == 0) {
    // G = inclusive prefix sum of g over the block (lanes past T add 0), and beta
    float gv = l < T ? graw : 0.f;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const float o = __shfl_up(gv, off, kWave);
      if (l >= off) gv += o;
    }
    if (l < TP) {
      sh.G[l] = gv;
      sh.beta[l] = l < T ? braw : 0.f;
    }
  }
  __syncthreads();

  // this wave's slice of St, loaded while step 2 runs (its barrier orders LDS only): column n of tile nt of
  // the B fragments is state row v = c0 + 16 nt + n, k = 32 kb + 8 (l / 16) .. + 8 contiguous in S[v][:]
  f32x4 sraw[4][2][2];
  {
    const float* sb = a.state + ((int64_t)b * a.Hv + h) * a.Dv * DK;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float* sr = sb + (int64_t)(c0 + nt * 16 + l % 16) * DK + (l / 16) * 8;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        sraw[kb][nt][0] = *reinterpret_cast<const f32x4*>(sr + kb * 32);
        sraw[kb][nt][1] = *reinterpret_cast<const f32x4*>(sr + kb * 32 + 4);
      }
    }
  }

  // ---- 2. K K^T (lower tiles) and Q K^T (all tiles) -> A (fp32) and M (bf16 hi + lo); the wave's LDS reads
  //         and MFMAs are all issued before its first store. The K rows go in as the A operand, so that each
  //         lane ends with 4 consecutive columns of one row: the layout of A's rows and of M's fragments
  const float GL = sh.G[T - 1];
  {
    constexpr int NKK = RT * (RT + 1) / 2, NJ = NKK + RT * RT, JPW = (NJ + NWV - 1) / NWV;
    f32x4 cj[JPW];
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = min(w + jj * NWV, NJ - 1);
      int ti, tj;
      job_tile<RT>(job, ti, tj);
      const uint16_t* X = job < NKK ? sh.K : sh.Q;
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < DK / 32; ++kb) {
        const u32x4 xa = *reinterpret_cast<const u32x4*>(&X[kq_off(ti * 16 + l % 16, kb * 4 + l / 16)]);
        const u32x4 kbv = *reinterpret_cast<const u32x4*>(&sh.K[kq_off(tj * 16 + l % 16, kb * 4 + l / 16)]);
        c = mma32(kbv, xa, c);
      }
      cj[jj] = c;
    }
#pragma unroll
    for (int jj = 0; jj < JPW; ++jj) {
      const int job = w + jj * NWV;
      if (job < NJ) {
        int ti, tj;
        job_tile<RT>(job, ti, tj);
        // cj holds row t = 16 ti + l % 16, columns s = 16 tj + 4 (l / 16) + i
        const int t = ti * 16 + l % 16, s0 = tj * 16 + (l / 16) * 4;
        const float Gt = sh.G[t];
        const f32x4 Gs = *reinterpret_cast<const f32x4*>(&sh.G[s0]);
        f32x4 r;
        if (job < NKK) {
          const float bt = sh.beta[t];
#pragma unroll
          for (int i = 0; i < 4; ++i) r[i] = s0 + i < t ? bt * cj[jj][i] * __expf(Gt - Gs[i]) : 0.f;
          sh.A[(ti * (ti + 1) / 2 + tj) * kWave + l] = r;
        } else {
          const bool causal = a.causal_mode == 1 || t < a.num_clean;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int s = s0 + i;
            if (causal) r[i] = s <= t ? cj[jj][i] * __expf(Gt - Gs[i]) : 0.f;
            else r[i] = s < T ? cj[jj][i] * __expf(GL - Gs[i]) : 0.f;
          }
          const uint32_t h01 = f2bf2(r.x, r.y), h23 = f2bf2(r.z, r.w);
          const uint32_t l01 = f2bf2(r.x - __uint_as_float(h01 << 16), r.y - __uint_as_float(h01 & 0xffff0000u));
          const uint32_t l23 = f2bf2(r.z - __uint_as_float(h23 << 16), r.w - __uint_as_float(h23 & 0xffff0000u));
          sh.M[(ti * RT + tj) * kWave + l] = u32x4{h01, h23, l01, l23};
        }
      }
    }
  }
  if (tid < TP) {
    const int t = tid;
    const bool causal = a.causal_mode == 1 || t < a.num_clean;
    sh.rs[t] = __expf(causal ? sh.G[t] : GL);
  }
  lds_barrier();

  // ---- 3. every wave: K St and Q St for its 32 columns (St hi + lo; K and Q exact), issued before the
  //         inverse so that the MFMAs run under its VALU work; the wave's V in the accumulator layout (rows
  //         4 (l / 16) + i, column l % 16; rows past T read row T - 1 and meet beta = 0) load meanwhile
  u32x4 sth[4][2], stl[4][2];  // St split into hi and lo
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) split8(sraw[kb][nt][0], sraw[kb][nt][1], sth[kb][nt], stl[kb][nt]);
  uint16_t vr[RT][2][4];
#pragma unroll
  for (int it = 0; it < RT; ++it)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = min(it * 16 + (l / 16) * 4 + i, T - 1);
      const uint16_t* vp = a.v + (((int64_t)b * T + t) * a.Hv + h) * a.Dv + c0 + l % 16;
      vr[it][0][i] = vp[0];
      vr[it][1][i] = vp[16];
    }
  f32x4 ks[RT][2], qs[RT][2];
#pragma unroll
  for (int it = 0; it < RT; ++it)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      ks[it][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
      qs[it][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
  for (int it = 0; it < RT; ++it)
#pragma unroll
    for (int kb = 0; kb < DK / 32; ++kb) {
      const u32x4 kf = *reinterpret_cast<const u32x4*>(&sh.K[kq_off(it * 16 + l % 16, kb * 4 + l / 16)]);
      const u32x4 qf = *reinterpret_cast<const u32x4*>(&sh.Q[kq_off(it * 16 + l % 16, kb * 4 + l / 16)]);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        ks[it][nt] = mma32(kf, sth[kb][nt], ks[it][nt]);
        ks[it][nt] = mma32(kf, stl[kb][nt], ks[it][nt]);
        qs[it][nt] = mma32(qf, sth[kb][nt], qs[it][nt]);
        qs[it][nt] = mma32(qf, stl[kb][nt], qs[it][nt]);
      }
    }
  // the diagonal 16 x 16 blocks of T = (I + A)^{-1} in fp32 by forward substitution, one block per wave
  // (lane j < 16 holds column j in registers): T[t][j] = [t == j] - sum_{s<t} A[t][s] T[s][j]
  for (int bi = w; bi < RT; bi += NWV) {
    const f32x4* ab = &sh.A[(bi * (bi + 1) / 2 + bi) * kWave];  // row t, columns s4 .. + 4: lane t + 4 s4
    float tc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};  // four independent chains (s mod 4), summed at the end
#pragma unroll
      for (int s4 = 0; s4 < t; s4 += 4) {
        const f32x4 ar = ab[t + 4 * s4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (s4 + e < t) acc[e] = fmaf(ar[e], tc[s4 + e], acc[e]);
      }
      tc[t] = (t == l % 16 ? 1.f : 0.f) - ((acc[0] + acc[1]) + (acc[2] + acc[3]));
    }
    if (l < 16) {
      float* tb = reinterpret_cast<float*>(&sh.Tm[bi * kWave]);
#pragma unroll
      for (int t = 0; t < 16; ++t) tb[(t + 4 * (l & ~3)) * 4 + (l & 3)] = tc[t];
    }
  }
  // R = diag(beta) (V - diag(e^G) K St), in the accumulator layout (the B operand of the 16x16x16 MFMA)
#pragma unroll
  for (int it = 0; it < RT; ++it)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = it * 16 + (l / 16) * 4 + i;
        ks[it][nt][i] = sh.beta[t] * (bf2f(vr[it][nt][i]) - __expf(sh.G[t]) * ks[it][nt][i]);
      }
  __syncthreads();

  // ---- 4. v_new by blocks: v_new_i = T[i][i] (R_i - sum_{k<i} A[i][k] v_new_k), then o = diag(rs) Q St + M v_new;
  //         each fp32 operand is split into hi + lo once
  s16x4 vh[RT][2], vl[RT][2];
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    s16x4 ah[RT], al[RT], th, tl;
#pragma unroll
    for (int k = 0; k < it; ++k) split4(sh.A[(it * (it + 1) / 2 + k) * kWave + l], ah[k], al[k]);
    split4(sh.Tm[it * kWave + l], th, tl);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      f32x4 x = ks[it][nt];
      if (it > 0) {
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < it; ++k) {
          c = mma16(ah[k], vh[k][nt], c);
          c = mma16(ah[k], vl[k][nt], c);
          c = mma16(al[k], vh[k][nt], c);
        }
        x -= c;
      }
      s16x4 xh, xl;
      split4(x, xh, xl);
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      v = mma16(th, xh, v);
      v = mma16(th, xl, v);
      v = mma16(tl, xh, v);
      split4(v, vh[it][nt], vl[it][nt]);
    }
  }
#pragma unroll
  for (int it = 0; it < RT; ++it) {
    s16x4 mh[RT], ml[RT];
#pragma unroll
    for (int kt = 0; kt < RT; ++kt) {
      const u32x4 mf = sh.M[(it * RT + kt) * kWave + l];
      mh[kt] = __builtin_bit_cast(s16x4, u32x2{mf.x, mf.y});
      ml[kt] = __builtin_bit_cast(s16x4, u32x2{mf.z, mf.w});
    }
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < RT; ++kt) {
        c = mma16(mh[kt], vh[kt][nt], c);
        c = mma16(mh[kt], vl[kt][nt], c);
        c = mma16(ml[kt], vh[kt][nt], c);
      }
      // into this wave's own columns of the output tile (K's LDS, unused since step 3): rows leave as
      // 16-byte pieces
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = it * 16 + (l / 16) * 4 + i;
        sh.K[t * NWV * CW + w * CW + nt * 16 + l % 16] = f2bf(a.scale * (sh.rs[t] * qs[it][nt][i] + c[i]));
      }
    }
  }
  // the wave's [TP][32] output: 4 lanes per row (64 bytes), rows < T (its own LDS writes land first)
#pragma unroll
  for (int j = 0; j < TP * 4 / kWave; ++j) {
    const int q = l + j * kWave, t = q / 4, part = q % 4;
    if (t < T) {
      uint16_t* dst = a.out + (((int64_t)b * T + t) * a.Hv + h) * a.Dv + c0 + part * 8;
      const uint16_t* src = &sh.K[t * NWV * CW + w * CW + part * 8];
      if ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
        *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
      } else {  // out is only 2-byte aligned
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = src[e];
      }
    }
  }
}

template <int NWV>
void launch_tp(const BlockArgs& a, int B, hipStream_t st) {
  const dim3 grid((unsigned)(B * a.Hv * (a.Dv / (NWV * CW))));
  const dim3 block(NWV * kWave);
  switch ((a.T + 15) / 16) {
    case 1: hipLaunchKernelGGL((gdr_block_kernel<16, NWV>), grid, block, 0, st, a); break;
    case 2: hipLaunchKernelGGL((gdr_block_kernel<32, NWV>), grid, block, 0, st, a); break;
    case 3: hipLaunchKernelGGL((gdr_block_kernel<48, NWV>), grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL((gdr_block_kernel<64, NWV>), grid, block, 0, st, a); break;
  }
}

}  // namespace

bool gdr_block_supported(int64_t T, int64_t Dk, int64_t Dv) { return T >= 1 && T <= 64 && Dk == DK && Dv % 128 == 0; }

int gdr_block_launch(const BlockArgs& a, int64_t B, hipStream_t stream) {
  // one workgroup per (sequence, head, 128 value columns): its 4 waves share the K K^T / Q K^T and
  // inverse work. At every grid size this beat one single-wave workgroup per 32 columns (which repeats
  // that work per wave): at one sequence of 33 rows x 16 heads 10.4 against 14.1 us
  launch_tp<4>(a, (int)B, stream);
  return launch_status("gdr_chunk/block");
}

}  // namespace trida
