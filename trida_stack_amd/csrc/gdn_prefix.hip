// Gated delta rule over a prefix of many chunks (T > 64 rows, Dk = 128) in two launches: a chunk-parallel
// preparation of every (sequence, chunk, value head) at once, then a scan per (sequence, value head, 16
// value columns) whose chain wave carries the state through the chunks in its registers.
//
// Per chunk (G_t = sum_{s<=t} g_s inside the chunk, L = the chunk's last row, St = S^T [Dk, Dv] at the
// chunk start; S as stored is [Dv, Dk]):
//   A[t][s] = beta_t (k_t . k_s) e^{G_t - G_s}   (s < t)        T = (I + A)^{-1}
//   M[t][s] = (q_t . k_s) e^{G_t - G_s}          (s <= t)
//   R       = diag(beta) (V - diag(e^G) K St)                  v_new = T R
//   o       = scale (diag(e^G) Q St + M v_new)
//   St'     = e^{G_L} St + K^T diag(e^{G_L - G}) v_new
// the chunk form of S = e^g S; S += beta (v - S k) k^T; o = S q. Rows past T enter as zeros (k = q = v = 0,
// g = beta = 0), which leaves St and every valid row unchanged. Every exponent taken is <= 0.
//
// Preparation (gdr_prefix_prep_kernel, 4 waves per (sequence, chunk, value head)): T in 16 x 16 blocks,
// D_i = (I + A_ii)^{-1} as the product (I + N)(I + N^2)(I + N^4)(I + N^8) of N = -A_ii (strictly lower
// triangular), then by columns T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj (T_ii = D_i); M from the Q K^T tiles.
// Both go to the workspace as the A fragments of the scan's products: T as bf16 hi + lo, M as bf16.
//
// Scan (gdr_prefix_scan_kernel, 8 waves per (sequence, value head, 16 value columns)): wave 0, the chain,
// keeps St (fp32, eight 16 x 16 tiles) in accumulator registers and runs K St, R, v_new = T R and the state
// update of chunk i with no barrier and no LDS round trip inside: each product's accumulators are the B
// operand of the next (see the slot order below). Waves 1, 2, 3 and 5 stage chunk i + 1 (K, K^T, V, the T
// fragments, the decays) into LDS while chunk i + 2 loads; waves 6-7 write the readout of chunk i - 1
// from the St and v_new fragments the chain left in LDS; wave 4 idles, so the chain has its SIMD to
// itself. One barrier per chunk.
//
// MFMA v_mfma_f32_16x16x32_bf16: A = row l % 16 with 8 k slots 8 (l / 16) + j; B = column l % 16 with the
// same slots; the accumulator holds rows 4 (l / 16) + e of column l % 16. A 32-wide k block covers the two
// 16-row tiles 2 kb and 2 kb + 1 with slot 8 g + j = row 32 kb + 4 g + j (j < 4) or 32 kb + 16 + 4 g + j - 4
// (j >= 4): the accumulators of the two tiles, side by side, are a B fragment as they stand. The A
// operands (K, K^T, T) are staged in this slot order, one 16-byte fragment per lane.
//
// Precision: fp32 operands enter the MFMAs as bf16 hi + lo with hi*hi + hi*lo + lo*hi (about 16 mantissa
// bits) where they feed the state (the state in K St, R, T, v_new in the state update, the inverse);
// bf16 inputs (k, q, v) enter exactly. Products that only feed the bf16 output (Q St, M v_new) take the
// bf16 rounding of their fp32 operand. Decays are e^x = 2^{x log2 e} on v_exp_f32 (G kept in log2 units).
// The inverse's 16 x 16 products run on v_mfma_f32_16x16x16_bf16 (A = row l % 16, k = 4 (l / 16) .. + 3;
// B = column l % 16, same k), whose accumulator layout is its own B layout.
#include <math.h>

#include "common.h"
#include "gdn_prefix.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int DK = 128;
constexpr int CH = 64;  // rows per chunk
constexpr int DS = 16;  // value columns per scan workgroup
constexpr int kPrepNT = 4 * kWave;
constexpr int kScanNT = 8 * kWave;
constexpr int TS = 68;  // bf16 row stride of T and M: 8-byte fragment reads of 16 rows hit distinct banks
constexpr int FS = 20;  // fp32 row stride of the 16 x 16 preparation tiles
// the (row tile, k block) pairs a lower-triangular 64 x 64 factor needs: (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
constexpr int kPairs = 6;
__device__ __forceinline__ int pair_it(int p) { return p < 2 ? p : 2 + (p - 2) / 2; }
__device__ __forceinline__ int pair_kb(int p) { return p < 2 ? 0 : (p - 2) % 2; }
// workspace per (sequence, chunk, value head) in 16-byte fragments (one per lane): T [pair][hi, lo][lane],
// M [pair][lane], then the decays beta, e^G, e^{G_L - G}, e^{G_L} as fp32 [4][64]
constexpr int kWsT = 0;
constexpr int kWsM = kPairs * 2 * kWave;
constexpr int kWsVec = kWsM + kPairs * kWave;
constexpr int kWsFrags = kWsVec + 4 * CH / 4;
static_assert(kWsFrags * 16 == kPrefixWsBytes, "prefix workspace layout");

__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ s16x4 as_s16(u32x2 v) { return __builtin_bit_cast(s16x4, v); }
__device__ __forceinline__ u32x2 ld2(const uint16_t* p) { return *reinterpret_cast<const u32x2*>(p); }
// two 4-slot halves -> one 8-slot fragment
__device__ __forceinline__ u32x4 cat2(u32x2 x, u32x2 y) { return u32x4{x.x, x.y, y.x, y.y}; }
__device__ __forceinline__ u32x4 cat(s16x4 a, s16x4 b) {
  return cat2(__builtin_bit_cast(u32x2, a), __builtin_bit_cast(u32x2, b));
}

// 4 fp32 -> bf16 hi + lo with x ~ hi + lo
__device__ __forceinline__ void split4(f32x4 x, s16x4& hi, s16x4& lo) {
  const uint32_t a = f2bf2(x[0], x[1]), b = f2bf2(x[2], x[3]);
  const uint32_t c = f2bf2(x[0] - __uint_as_float(a << 16), x[1] - __uint_as_float(a & 0xffff0000u));
  const uint32_t d = f2bf2(x[2] - __uint_as_float(b << 16), x[3] - __uint_as_float(b & 0xffff0000u));
  hi = as_s16(u32x2{a, b});
  lo = as_s16(u32x2{c, d});
}
__device__ __forceinline__ s16x4 hi4(f32x4 x) { return as_s16(u32x2{f2bf2(x[0], x[1]), f2bf2(x[2], x[3])}); }
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ f32x4 mm3(s16x4 ah, s16x4 al, s16x4 bh, s16x4 bl, f32x4 c) {
  c = mma16(ah, bh, c);
  c = mma16(ah, bl, c);
  return mma16(al, bh, c);
}
__device__ __forceinline__ f32x4 mm3x(u32x4 ah, u32x4 al, u32x4 bh, u32x4 bl, f32x4 c) {
  c = mma32(ah, bh, c);
  c = mma32(ah, bl, c);
  return mma32(al, bh, c);
}

// K / Q rows [CH][DK] bf16 of the preparation: 16-byte groups XOR-swizzled by the row
__device__ __forceinline__ int kq_off(int r, int grp) { return r * DK + ((grp ^ (r & 15)) << 3); }

__device__ __forceinline__ void lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// workgroup barrier over LDS only: global loads stay in flight across it
__device__ __forceinline__ void bar() {
  lds_order();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// inclusive prefix sum over the 64 lanes (one chunk row per lane), in log2 units
__device__ __forceinline__ float chunk_g2(float g, int l) {
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const float o = __shfl_up(g, off, kWave);
    if (l >= off) g += o;
  }
  return g * kLog2e;
}

// ==================================================================== preparation
struct PrepLds {
  uint16_t K[CH * DK];
  uint16_t Q[CH * DK];
  float G2[CH], be[CH];  // G log2(e), beta
  uint16_t Th[CH * TS], Tl[CH * TS], Mh[CH * TS];
  __align__(16) float Dd[4][16 * FS];  // inverses of the diagonal blocks, row-major fp32
  u32x2 Ao[6][2][kWave];               // off-diagonal A tiles (1,0) (2,0) (2,1) (3,0) (3,1) (3,2) as A
                                       // fragments, hi and lo
};

// A operand of a 16 x 16 fp32 tile stored row-major (stride FS): row l % 16, k = 4 (l / 16) .. + 3
__device__ __forceinline__ void a_frag(const float* X, int l, s16x4& h, s16x4& lo) {
  split4(*reinterpret_cast<const f32x4*>(&X[(l % 16) * FS + 4 * (l / 16)]), h, lo);
}
// B operand of the same storage: X[4 (l / 16) + r][l % 16]
__device__ __forceinline__ void b_frag(const float* X, int l, s16x4& h, s16x4& lo) {
  f32x4 x;
#pragma unroll
  for (int r = 0; r < 4; ++r) x[r] = X[(4 * (l / 16) + r) * FS + l % 16];
  split4(x, h, lo);
}
// X Y with X a row-major fp32 tile and Y given as B fragments hi / lo
__device__ __forceinline__ f32x4 prod(const float* X, s16x4 yh, s16x4 yl, f32x4 c, int l) {
  s16x4 xh, xl;
  a_frag(X, l, xh, xl);
  return mm3(xh, xl, yh, yl, c);
}
// A_ik Y with A_ik given as stored A fragments
__device__ __forceinline__ f32x4 prod_ao(const PrepLds& sh, int idx, s16x4 yh, s16x4 yl, f32x4 c, int l) {
  return mm3(as_s16(sh.Ao[idx][0][l]), as_s16(sh.Ao[idx][1][l]), yh, yl, c);
}
// -D_i Y (Y in accumulator layout)
__device__ __forceinline__ f32x4 neg_d(const float* D, f32x4 y, int l) {
  s16x4 yh, yl;
  split4(y, yh, yl);
  const f32x4 r = prod(D, yh, yl, f32x4{0.f, 0.f, 0.f, 0.f}, l);
  return -r;
}
// a T tile (accumulator layout) -> Th / Tl
__device__ __forceinline__ void put_t(PrepLds& sh, int ti, int tj, f32x4 x, int l) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int o = (16 * ti + 4 * (l / 16) + r) * TS + 16 * tj + l % 16;
    const uint16_t h = f2bf(x[r]);
    sh.Th[o] = h;
    sh.Tl[o] = f2bf(x[r] - bf2f(h));
  }
}
// K K^T or Q K^T tile (rows 16 ti of X, columns 16 tj of K) in accumulator layout
__device__ __forceinline__ f32x4 xk_tile(const uint16_t* X, const uint16_t* Kc, int ti, int tj, int l) {
  f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kb = 0; kb < DK / 32; ++kb) {
    const u32x4 xa = *reinterpret_cast<const u32x4*>(&X[kq_off(16 * ti + l % 16, 4 * kb + l / 16)]);
    const u32x4 kf = *reinterpret_cast<const u32x4*>(&Kc[kq_off(16 * tj + l % 16, 4 * kb + l / 16)]);
    c = mma32(xa, kf, c);
  }
  return c;
}

// wave pw: the diagonal block pw and its inverse, and its share of the off-diagonal A tiles
__device__ __forceinline__ void prep_blocks(PrepLds& sh, int pw, int l) {
  const uint16_t* Kc = sh.K;
  const float* G2 = sh.G2;
  const float* be = sh.be;
  const int r = l % 16, q4 = 4 * (l / 16);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  // N = -A_pp in both operand layouts from the one (symmetric) K K^T tile, then
  // D = (I - N)^{-1} = (I + N)(I + N^2)(I + N^4)(I + N^8) (N is strictly lower triangular, N^16 = 0).
  // The accumulator layout of X^T is the A layout of X, and the factors commute, so every product takes
  // both operands from registers.
  {
    const f32x4 cd = xk_tile(Kc, Kc, pw, pw, l);
    const int p0 = 16 * pw;
    const float Gr = G2[p0 + r], br = be[p0 + r];
    f32x4 nc, na;
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // branch-free: decays clamped to <= 0 where masked out
      const int t = q4 + e;
      const float gt = G2[p0 + t], bt = be[p0 + t];
      const float xc = -bt * cd[e] * ex2(fminf(gt - Gr, 0.f));
      const float xa = -br * cd[e] * ex2(fminf(Gr - gt, 0.f));
      nc[e] = r < t ? xc : 0.f;  // N[t][r]
      na[e] = t < r ? xa : 0.f;  // N[r][t]
    }
    s16x4 nah, nal, nch, ncl;
    split4(na, nah, nal);
    split4(nc, nch, ncl);
    const f32x4 n2c = mm3(nah, nal, nch, ncl, z);  // N^2
    const f32x4 n2a = mm3(nch, ncl, nah, nal, z);  // (N^2)^T
    s16x4 n2ah, n2al, n2ch, n2cl;
    split4(n2a, n2ah, n2al);
    split4(n2c, n2ch, n2cl);
    const f32x4 n4c = mm3(n2ah, n2al, n2ch, n2cl, z);
    const f32x4 n4a = mm3(n2ch, n2cl, n2ah, n2al, z);
    s16x4 n4ah, n4al, n4ch, n4cl;
    split4(n4a, n4ah, n4al);
    split4(n4c, n4ch, n4cl);
    const f32x4 n8a = mm3(n4ch, n4cl, n4ah, n4al, z);  // (N^8)^T
    s16x4 n8ah, n8al;
    split4(n8a, n8ah, n8al);
    f32x4 d = nc;
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] += (q4 + e == r) ? 1.f : 0.f;
    s16x4 dh, dl;
    split4(d, dh, dl);
    d = mm3(n2ah, n2al, dh, dl, d);
    split4(d, dh, dl);
    d = mm3(n4ah, n4al, dh, dl, d);
    split4(d, dh, dl);
    d = mm3(n8ah, n8al, dh, dl, d);
#pragma unroll
    for (int e = 0; e < 4; ++e) sh.Dd[pw][(q4 + e) * FS + r] = d[e];
  }
  // Off-diagonal A tiles (wave 0: (1,0) (2,0); 1: (2,1) (3,0); 2: (3,1); 3: (3,2)), each from the
  // transposed K K^T tile, whose accumulator layout is the A layout of the (ti, tj) tile
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int idx = pw < 2 ? 2 * pw + j : (j == 0 ? pw + 2 : -1);
    if (idx >= 0) {
      const int ti = idx == 0 ? 1 : idx < 3 ? 2 : 3;
      const int tj = idx == 0 ? 0 : idx < 3 ? idx - 1 : idx - 3;
      const f32x4 ct = xk_tile(Kc, Kc, tj, ti, l);
      const int row = 16 * ti + r;
      const float Gr = G2[row], br = be[row];
      f32x4 av;
#pragma unroll
      for (int e = 0; e < 4; ++e) av[e] = br * ct[e] * ex2(Gr - G2[16 * tj + q4 + e]);
      s16x4 hh, ll;
      split4(av, hh, ll);
      sh.Ao[idx][0][l] = __builtin_bit_cast(u32x2, hh);
      sh.Ao[idx][1][l] = __builtin_bit_cast(u32x2, ll);
    }
  }
}

// wave pw: one column chain of T (pw = 0..2) or the diagonal tiles (pw = 3)
__device__ __forceinline__ void prep_columns(PrepLds& sh, int pw, int l) {
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  if (pw == 0) {  // column 0: T10, T20, T30
    s16x4 dh, dl;
    b_frag(sh.Dd[0], l, dh, dl);
    const f32x4 t10 = neg_d(sh.Dd[1], prod_ao(sh, 0, dh, dl, z, l), l);
    s16x4 h10, l10;
    split4(t10, h10, l10);
    const f32x4 t20 = neg_d(sh.Dd[2], prod_ao(sh, 2, h10, l10, prod_ao(sh, 1, dh, dl, z, l), l), l);
    s16x4 h20, l20;
    split4(t20, h20, l20);
    const f32x4 y3 = prod_ao(sh, 5, h20, l20, prod_ao(sh, 4, h10, l10, prod_ao(sh, 3, dh, dl, z, l), l), l);
    const f32x4 t30 = neg_d(sh.Dd[3], y3, l);
    put_t(sh, 1, 0, t10, l);
    put_t(sh, 2, 0, t20, l);
    put_t(sh, 3, 0, t30, l);
  } else if (pw == 1) {  // column 1: T21, T31
    s16x4 dh, dl;
    b_frag(sh.Dd[1], l, dh, dl);
    const f32x4 t21 = neg_d(sh.Dd[2], prod_ao(sh, 2, dh, dl, z, l), l);
    s16x4 h21, l21;
    split4(t21, h21, l21);
    const f32x4 t31 = neg_d(sh.Dd[3], prod_ao(sh, 5, h21, l21, prod_ao(sh, 4, dh, dl, z, l), l), l);
    put_t(sh, 2, 1, t21, l);
    put_t(sh, 3, 1, t31, l);
  } else if (pw == 2) {  // column 2: T32
    s16x4 dh, dl;
    b_frag(sh.Dd[2], l, dh, dl);
    put_t(sh, 3, 2, neg_d(sh.Dd[3], prod_ao(sh, 5, dh, dl, z, l), l), l);
  } else {  // the diagonal tiles T_ii = D_i
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s16x4 hh, ll;
      split4(*reinterpret_cast<const f32x4*>(&sh.Dd[i][(l / 4) * FS + 4 * (l % 4)]), hh, ll);
      const int o = (16 * i + l / 4) * TS + 16 * i + 4 * (l % 4);
      *reinterpret_cast<u32x2*>(&sh.Th[o]) = __builtin_bit_cast(u32x2, hh);
      *reinterpret_cast<u32x2*>(&sh.Tl[o]) = __builtin_bit_cast(u32x2, ll);
    }
  }
}

// Q K^T tiles (lower triangle, 10 tiles; wave w takes tiles w, w + 4, w + 8) -> M (bf16)
__device__ __forceinline__ void prep_m(PrepLds& sh, int w, int l) {
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int idx = w + 4 * j;
    if (idx < 10) {
      const int ti = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
      const int tj = idx - ti * (ti + 1) / 2;
      const f32x4 cq = xk_tile(sh.Q, sh.K, ti, tj, l);
      const int s = 16 * tj + l % 16;
      const float Gs = sh.G2[s];
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // branch-free: the decay is clamped to <= 0 where it is masked out
        const int t = 16 * ti + 4 * (l / 16) + e;
        const float x = cq[e] * ex2(fminf(sh.G2[t] - Gs, 0.f));
        sh.Mh[t * TS + s] = f2bf(s <= t ? x : 0.f);
      }
    }
  }
}

template <bool OUT>
__global__ __launch_bounds__(kPrepNT) void gdr_prefix_prep_kernel(PrefixArgs a) {
  __shared__ __align__(16) PrepLds sh;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), l = threadIdx.x % kWave;
  int idx = blockIdx.x;  // (sequence, chunk, value head), heads innermost
  const int h = idx % a.Hv;
  idx /= a.Hv;
  const int c = idx % a.nchunks, b = idx / a.nchunks;
  const int hk = h / (a.Hv / a.Hk);
  const int t0 = c * CH;
  // K (and Q) rows 16 w + 4 (l / 16) + u, columns 8 (l % 16) .. + 7; rows past T read row 0 (in bounds)
  // and are zeroed after the load
  u32x4 kr[4], qr[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 16 * w + 4 * (l / 16) + u;
    const bool ok = t < a.T;
    const int64_t off = ((int64_t)(b * a.T + (ok ? t : 0)) * a.Hk + hk) * DK + 8 * (l % 16);
    const u32x4 kv = *reinterpret_cast<const u32x4*>(a.k + off);
    kr[u] = ok ? kv : u32x4{0u, 0u, 0u, 0u};
    if (OUT) {
      const u32x4 qv = *reinterpret_cast<const u32x4*>(a.q + off);
      qr[u] = ok ? qv : u32x4{0u, 0u, 0u, 0u};
    }
  }
  float gv = 0.f, bv = 0.f;
  if (w == 0) {
    const int t = t0 + l;
    const bool ok = t < a.T;
    const int64_t gi = (int64_t)(b * a.T + (ok ? t : 0)) * a.Hv + h;
    const float x = a.g[gi], y = a.beta[gi];
    gv = ok ? x : 0.f;
    bv = ok ? y : 0.f;
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int o = kq_off(16 * w + 4 * (l / 16) + u, l % 16);
    *reinterpret_cast<u32x4*>(&sh.K[o]) = kr[u];
    if (OUT) *reinterpret_cast<u32x4*>(&sh.Q[o]) = qr[u];
  }
  u32x4* dst = static_cast<u32x4*>(a.ws) + ((int64_t)(b * a.nchunks + c) * a.Hv + h) * kWsFrags;
  if (w == 0) {
    const float G = chunk_g2(gv, l);
    const float GL = __shfl(G, kWave - 1, kWave);
    sh.G2[l] = G;
    sh.be[l] = bv;
    float* vec = reinterpret_cast<float*>(dst + kWsVec);  // the scan's decays
    vec[l] = bv;
    vec[CH + l] = ex2(G);
    vec[2 * CH + l] = ex2(GL - G);
    vec[3 * CH + l] = ex2(GL);
  }
  bar();
  prep_blocks(sh, w, l);
  bar();
  prep_columns(sh, w, l);
  if (OUT) prep_m(sh, w, l);
  bar();
  // the fragments: pair (it, kb) holds rows 16 it + l % 16 at k slots 32 kb + 4 g .. + 3 and 32 kb + 16 +
  // 4 g .. + 3 (g = l / 16); the tiles above the diagonal are zero
  for (int p = w; p < kPairs; p += 4) {
    const int it = pair_it(p), kb = pair_kb(p);
    const int o = (16 * it + l % 16) * TS + 32 * kb + 4 * (l / 16);
    const bool up0 = 2 * kb > it, up1 = 2 * kb + 1 > it;
    const u32x2 zz = {0u, 0u};
    dst[kWsT + (2 * p) * kWave + l] = cat2(up0 ? zz : ld2(&sh.Th[o]), up1 ? zz : ld2(&sh.Th[o + 16]));
    dst[kWsT + (2 * p + 1) * kWave + l] = cat2(up0 ? zz : ld2(&sh.Tl[o]), up1 ? zz : ld2(&sh.Tl[o + 16]));
    if (OUT) dst[kWsM + p * kWave + l] = cat2(up0 ? zz : ld2(&sh.Mh[o]), up1 ? zz : ld2(&sh.Mh[o + 16]));
  }
}

// ==================================================================== scan
// The staged K and K^T fragments keep lane ln's 16 bytes in slot ln ^ 2 j ^ (ln >> 5 & 1) (K St, k block
// j) and ln ^ m (state update, Dk tile m): the staging writes, 8 bytes from each lane, then spread over the
// LDS banks instead of landing on a few of them.
__device__ __forceinline__ int kf_slot(int ln, int j) { return ln ^ (2 * j) ^ ((ln >> 5) & 1); }
__device__ __forceinline__ int ktf_slot(int ln, int m) { return ln ^ (m & 7); }

struct ScanLds {
  // K as the A fragments of K St: [row tile][k block][slot], and K^T as those of the state update:
  // [Dk tile][k block][slot] (buffer = chunk parity)
  u32x4 Kf[2][4][4][kWave];
  u32x4 KTf[2][8][2][kWave];
  u32x4 T[2][kPairs][2][kWave];     // T fragments hi / lo, as in the workspace
  u32x2 V[2][4][kWave];             // this workgroup's value columns in accumulator layout [row tile][lane]
  float vec[3][4][CH];              // beta, e^G, e^{G_L - G}, e^{G_L} (every entry); buffer = chunk mod 3
  u32x4 xS[2][4][kWave];            // St hi at the chunk start as B fragments per k block (readout)
  u32x4 xV[2][2][kWave];            // v_new hi as B fragments per k block (readout)
  uint16_t xO[CH][DS];              // the readout's rows, transposed for 16-byte row stores
};
static_assert(sizeof(ScanLds) <= 160 * 1024, "LDS plan exceeds 160 KiB");

// what a staging wave pw (0..3) loads for one chunk: K rows 16 pw + 4 (l / 16) + u, columns 8 (l % 16) ..
// + 7; the V row 16 pw + l / 4, columns 4 (l % 4) .. + 3 of this workgroup's slice; the T fragments
// 256 j + 64 pw + l; decay entry 64 pw + l. Rows past T read row 0 (in bounds) and are zeroed when staged:
// nothing consumes a load until the next iteration, so the loads stay in flight across the barrier
struct Raw {
  u32x4 k[4];
  u32x4 t[3];
  u32x2 v;
  float dec;
};

__device__ __forceinline__ void load_raw(Raw& r, const PrefixArgs& a, int b, int h, int hk, int dv0, int c, int pw,
                                         int l) {
  const int t0 = c * CH;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 16 * pw + 4 * (l / 16) + u;
    const int64_t off = ((int64_t)(b * a.T + (t < a.T ? t : 0)) * a.Hk + hk) * DK + 8 * (l % 16);
    r.k[u] = *reinterpret_cast<const u32x4*>(a.k + off);
  }
  {
    const int t = t0 + 16 * pw + l / 4;
    const int64_t off = ((int64_t)(b * a.T + (t < a.T ? t : 0)) * a.Hv + h) * a.Dv + dv0 + 4 * (l % 4);
    r.v = *reinterpret_cast<const u32x2*>(a.v + off);
  }
  const u32x4* src = static_cast<const u32x4*>(a.ws) + ((int64_t)(b * a.nchunks + c) * a.Hv + h) * kWsFrags;
#pragma unroll
  for (int j = 0; j < 3; ++j) r.t[j] = src[kWsT + 256 * j + 64 * pw + l];
  r.dec = reinterpret_cast<const float*>(src + kWsVec)[64 * pw + l];
}

__device__ __forceinline__ void stage(ScanLds& sh, const Raw& r, int T, int c, int pw, int l) {
  const int kb = c & 1, g = l / 16, cg = l % 16;
  u32x4 k[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) k[u] = c * CH + 16 * pw + 4 * g + u < T ? r.k[u] : u32x4{0u, 0u, 0u, 0u};
  // The lane holds K[16 pw + 4 g + u][8 cg + e] (u = 0..3, e = 0..7). In the K St fragments (row tile pw,
  // k block cg / 4) its elements e = 0..3 and 4..7 of row u are the halves (cg % 4) / 2 of lanes
  // 16 (2 (cg % 2)) + 4 g + u and 16 (2 (cg % 2) + 1) + 4 g + u
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    uint16_t* f = reinterpret_cast<uint16_t*>(&sh.Kf[kb][pw][cg / 4][0]) + 4 * ((cg % 4) / 2);
    const int ln = 16 * (2 * (cg % 2)) + 4 * g + u;
    *reinterpret_cast<u32x2*>(f + 8 * kf_slot(ln, cg / 4)) = u32x2{k[u][0], k[u][1]};
    *reinterpret_cast<u32x2*>(f + 8 * kf_slot(ln + 16, cg / 4)) = u32x2{k[u][2], k[u][3]};
  }
  // In the state update's K^T fragments (Dk tile cg / 2, k block pw / 2) rows u = 0..3 of column 8 cg + e
  // are the half pw % 2 of lane 16 g + 8 (cg % 2) + e
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint32_t x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) x[u] = (k[u][e >> 1] >> (16 * (e & 1))) & 0xffffu;
    uint16_t* f = reinterpret_cast<uint16_t*>(&sh.KTf[kb][cg / 2][pw / 2][0]) + 4 * (pw % 2);
    *reinterpret_cast<u32x2*>(f + 8 * ktf_slot(16 * g + 8 * (cg % 2) + e, cg / 2)) =
        u32x2{x[0] | (x[1] << 16), x[2] | (x[3] << 16)};
  }
  // V[16 pw + tt][4 (l % 4) + cc] (tt = l / 4) -> tile pw, lane 16 (tt / 4) + 4 (l % 4) + cc, element tt % 4
  {
    uint16_t* vt = reinterpret_cast<uint16_t*>(&sh.V[kb][pw][0]);
    const int tt = l / 4;
    const u32x2 vv = c * CH + 16 * pw + tt < T ? r.v : u32x2{0u, 0u};
    const uint16_t e4[4] = {(uint16_t)(vv.x & 0xffffu), (uint16_t)(vv.x >> 16), (uint16_t)(vv.y & 0xffffu),
                            (uint16_t)(vv.y >> 16)};
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) vt[(16 * (tt / 4) + 4 * (l % 4) + cc) * 4 + tt % 4] = e4[cc];
  }
  u32x4* tf = &sh.T[kb][0][0][0];
#pragma unroll
  for (int j = 0; j < 3; ++j) tf[256 * j + 64 * pw + l] = r.t[j];
  (&sh.vec[c % 3][0][0])[64 * pw + l] = r.dec;
}

// the chain's step on chunk i: St (accumulators st, B fragments sh_ / sl_) -> St'
__device__ __forceinline__ void chain_step(ScanLds& sh, int i, int l, f32x4 (&st)[8], u32x4 (&sbh)[4],
                                           u32x4 (&sbl)[4]) {
  const int kb = i & 1, vb = i % 3, g4 = 4 * (l / 16);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  // the state at the chunk start (hi) for the readout of this chunk
#pragma unroll
  for (int j = 0; j < 4; ++j) sh.xS[kb][j][l] = sbh[j];
  // K St: row tile it, k block j (Dk rows 32 j ..), St hi and lo
  f32x4 ks[4] = {z, z, z, z};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const u32x4 ka = sh.Kf[kb][it][j][kf_slot(l, j)];
      ks[it] = mma32(ka, sbh[j], ks[it]);
      ks[it] = mma32(ka, sbl[j], ks[it]);
    }
  }
  // R = diag(beta) (V - diag(e^G) K St), rows 16 it + 4 (l / 16) + e
  s16x4 rh[4], rl[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const f32x4 be4 = *reinterpret_cast<const f32x4*>(&sh.vec[vb][0][16 * it + g4]);
    const f32x4 eg4 = *reinterpret_cast<const f32x4*>(&sh.vec[vb][1][16 * it + g4]);
    const u32x2 vv = sh.V[kb][it][l];
    const float v4[4] = {__uint_as_float(vv.x << 16), __uint_as_float(vv.x & 0xffff0000u),
                         __uint_as_float(vv.y << 16), __uint_as_float(vv.y & 0xffff0000u)};
    f32x4 R;
#pragma unroll
    for (int e = 0; e < 4; ++e) R[e] = be4[e] * (v4[e] - eg4[e] * ks[it][e]);
    split4(R, rh[it], rl[it]);
  }
  const u32x4 rbh0 = cat(rh[0], rh[1]), rbl0 = cat(rl[0], rl[1]);
  const u32x4 rbh1 = cat(rh[2], rh[3]), rbl1 = cat(rl[2], rl[3]);
  // v_new = T R over the pairs (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
  f32x4 vn[4];
  vn[0] = mm3x(sh.T[kb][0][0][l], sh.T[kb][0][1][l], rbh0, rbl0, z);
  vn[1] = mm3x(sh.T[kb][1][0][l], sh.T[kb][1][1][l], rbh0, rbl0, z);
  vn[2] = mm3x(sh.T[kb][3][0][l], sh.T[kb][3][1][l], rbh1, rbl1,
               mm3x(sh.T[kb][2][0][l], sh.T[kb][2][1][l], rbh0, rbl0, z));
  vn[3] = mm3x(sh.T[kb][5][0][l], sh.T[kb][5][1][l], rbh1, rbl1,
               mm3x(sh.T[kb][4][0][l], sh.T[kb][4][1][l], rbh0, rbl0, z));
  // v_new hi for the readout
  sh.xV[kb][0][l] = cat(hi4(vn[0]), hi4(vn[1]));
  sh.xV[kb][1][l] = cat(hi4(vn[2]), hi4(vn[3]));
  // St' = e^{G_L} St + K^T diag(e^{G_L - G}) v_new on the eight Dk tiles
  s16x4 ph[4], pl[4];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(&sh.vec[vb][2][16 * it + g4]);
    f32x4 vp;
#pragma unroll
    for (int e = 0; e < 4; ++e) vp[e] = vn[it][e] * d4[e];
    split4(vp, ph[it], pl[it]);
  }
  const u32x4 pbh0 = cat(ph[0], ph[1]), pbl0 = cat(pl[0], pl[1]);
  const u32x4 pbh1 = cat(ph[2], ph[3]), pbl1 = cat(pl[2], pl[3]);
  const float eL = sh.vec[vb][3][0];
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    f32x4 s;
#pragma unroll
    for (int e = 0; e < 4; ++e) s[e] = st[m][e] * eL;
    const u32x4 k0 = sh.KTf[kb][m][0][ktf_slot(l, m)], k1 = sh.KTf[kb][m][1][ktf_slot(l, m)];
    s = mma32(k0, pbh0, s);
    s = mma32(k0, pbl0, s);
    s = mma32(k1, pbh1, s);
    s = mma32(k1, pbl1, s);
    st[m] = s;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    s16x4 h0, l0, h1, l1;
    split4(st[2 * j], h0, l0);
    split4(st[2 * j + 1], h1, l1);
    sbh[j] = cat(h0, h1);
    sbl[j] = cat(l0, l1);
  }
}

template <bool OUT>
__global__ __launch_bounds__(kScanNT) void gdr_prefix_scan_kernel(PrefixArgs a) {
  __shared__ __align__(16) ScanLds sh;
  const int slices = a.Dv / DS;
  int idx = xcd_major(blockIdx.x, gridDim.x);  // a head's value slices (same K rows and T) on one XCD
  const int sl = idx % slices;
  idx /= slices;
  const int b = idx / a.Hv, h = idx % a.Hv, hk = h / (a.Hv / a.Hk), dv0 = sl * DS;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), l = threadIdx.x % kWave;
  const int n = a.nchunks;
  // Every wave runs the same n + 2 iterations with one barrier each. Iteration i: the chain on chunk i,
  // the staging of chunk i + 1 (and the loads of chunk i + 2), the readout of chunk i - 1.
  if (w == 0) {
    f32x4 st[8];
    u32x4 sbh[4], sbl[4];
    const int64_t soff = (((int64_t)b * a.Hv + h) * a.Dv + dv0 + l % 16) * DK + 4 * (l / 16);
#pragma unroll
    for (int m = 0; m < 8; ++m) st[m] = *reinterpret_cast<const f32x4*>(a.state_in + soff + 16 * m);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s16x4 h0, l0, h1, l1;
      split4(st[2 * j], h0, l0);
      split4(st[2 * j + 1], h1, l1);
      sbh[j] = cat(h0, h1);
      sbl[j] = cat(l0, l1);
    }
    for (int i = -1; i <= n; ++i) {
      if (i >= 0 && i < n) chain_step(sh, i, l, st, sbh, sbl);
      bar();
    }
    if (a.state_out) {
#pragma unroll
      for (int m = 0; m < 8; ++m) *reinterpret_cast<f32x4*>(a.state_out + soff + 16 * m) = st[m];
    }
  } else if (w != 4 && w < 6) {
    const int pw = w < 4 ? w - 1 : 3;
    Raw r;
    load_raw(r, a, b, h, hk, dv0, 0, pw, l);
    for (int i = -1; i <= n; ++i) {
      const int c = i + 1;
      if (c < n) {
        stage(sh, r, a.T, c, pw, l);
        if (c + 1 < n) load_raw(r, a, b, h, hk, dv0, c + 1, pw, l);
      }
      bar();
    }
  } else if (OUT && w >= 6) {
    // row tiles 2 (w - 6) and 2 (w - 6) + 1 of each chunk: Q and M fragments load one iteration ahead
    const int g4 = 4 * (l / 16);
    const int64_t vrow = (int64_t)a.Hv * a.Dv;
    u32x4 qf[2][4], mf[2][2];
    for (int i = -1; i <= n; ++i) {
      if (i >= 1) {
        const int c = i - 1, kb = c & 1, vb = c % 3;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int rt = 2 * (w - 6) + tt;
          f32x4 qs = {0.f, 0.f, 0.f, 0.f}, mv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < 4; ++j) qs = mma32(qf[tt][j], sh.xS[kb][j][l], qs);
          mv = mma32(mf[tt][0], sh.xV[kb][0][l], mv);
          if (rt >= 2) mv = mma32(mf[tt][1], sh.xV[kb][1][l], mv);
          const f32x4 eg4 = *reinterpret_cast<const f32x4*>(&sh.vec[vb][1][16 * rt + g4]);
#pragma unroll
          for (int e = 0; e < 4; ++e) sh.xO[16 * rt + g4 + e][l % 16] = f2bf(a.scale * (eg4[e] * qs[e] + mv[e]));
        }
        // this wave's 32 rows, half a row (16 bytes) per lane (its own LDS writes above land first); 2-byte
        // stores when out is not 16-byte aligned
        const int r = 32 * (w - 6) + l / 2, tg = c * CH + r;
        if (tg < a.T) {
          uint16_t* orow = a.out + ((int64_t)b * a.T + tg) * vrow + (int64_t)h * a.Dv + dv0 + 8 * (l % 2);
          if ((reinterpret_cast<uintptr_t>(a.out) & 15) == 0) {
            *reinterpret_cast<u32x4*>(orow) = *reinterpret_cast<const u32x4*>(&sh.xO[r][8 * (l % 2)]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) orow[e] = sh.xO[r][8 * (l % 2) + e];
          }
        }
      }
      if (i >= 0 && i < n) {
        const u32x4* mw = static_cast<const u32x4*>(a.ws) + ((int64_t)(b * n + i) * a.Hv + h) * kWsFrags + kWsM;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int rt = 2 * (w - 6) + tt;
          const int t = min(i * CH + 16 * rt + l % 16, a.T - 1);  // rows past T: computed, never stored
          const uint16_t* qrow = a.q + ((int64_t)(b * a.T + t) * a.Hk + hk) * DK;
#pragma unroll
          for (int j = 0; j < 4; ++j) qf[tt][j] = cat2(ld2(qrow + 32 * j + g4), ld2(qrow + 32 * j + 16 + g4));
          mf[tt][0] = mw[(rt < 2 ? rt : 2 + 2 * (rt - 2)) * kWave + l];
          if (rt >= 2) mf[tt][1] = mw[(3 + 2 * (rt - 2)) * kWave + l];
        }
      }
      bar();
    }
  } else {
    for (int i = -1; i <= n; ++i) bar();
  }
}

}  // namespace

bool gdr_prefix_supported(int64_t B, int64_t T, int64_t Hv, int64_t Dk, int64_t Dv) {
  // one scan workgroup per CU at most: the scan is latency-bound per chunk, and a grid of several rounds
  // runs its chunk chains one round after the other (larger batches take the prep + scan kernels of the
  // general chunked path)
  return T > CH && Dk == DK && Dv % DS == 0 && B * Hv * (Dv / DS) <= 256;
}

int gdr_prefix_launch(const PrefixArgs& a, int64_t B, hipStream_t stream) {
  const dim3 pgrid((unsigned)(B * a.nchunks * a.Hv));
  if (a.out) hipLaunchKernelGGL(gdr_prefix_prep_kernel<true>, pgrid, dim3(kPrepNT), 0, stream, a);
  else hipLaunchKernelGGL(gdr_prefix_prep_kernel<false>, pgrid, dim3(kPrepNT), 0, stream, a);
  int rc = launch_status("gdr_chunk/prefix prep");
  if (rc) return rc;
  const dim3 grid((unsigned)(B * a.Hv * (a.Dv / DS)));
  if (a.out) hipLaunchKernelGGL(gdr_prefix_scan_kernel<true>, grid, dim3(kScanNT), 0, stream, a);
  else hipLaunchKernelGGL(gdr_prefix_scan_kernel<false>, grid, dim3(kScanNT), 0, stream, a);
  return launch_status("gdr_chunk/prefix scan");
}

}  // namespace trida
