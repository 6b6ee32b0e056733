// Gated delta rule over a prefix of many chunks (T > 64 rows, Dk = 128) in one launch: per (sequence,
// value head, 16 value columns) one workgroup walks the 64-row chunks in order, the preparation of chunk
// c + 1 running beside the state recurrence of chunk c. No workspace: every intermediate stays in LDS.
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
// T is built in 16 x 16 blocks: D_i = (I + A_ii)^{-1} as the product (I + N)(I + N^2)(I + N^4)(I + N^8) of
// N = -A_ii (strictly lower triangular), then by columns T_ij = -D_i sum_{k=j}^{i-1} A_ik T_kj (T_ii = D_i).
//
// Workgroup = 8 waves. Waves 0-3 (the chain) own row tile w of a chunk for K St, Q St, R and o, and Dk
// tiles 2w, 2w+1 of the state (fp32, in accumulator registers from the first chunk to the last); waves
// 4-7 (the preparation) own row tile w - 4 of a chunk for its loads and LDS staging. Iteration i runs the
// chain on chunk i and the preparation on chunk i + 1 in three phases separated by barriers:
//   A  chain: K St and Q St (state fragments from LDS), R -> LDS
//      prep:  K, Q, K^T and V rows, G, beta and the decays -> LDS (two buffers each); loads of chunk i + 2
//   B  chain: v_new = T R (every row tile), o of its row tile, its two state tiles updated -> LDS
//      prep:  the diagonal A tile and its inverse D_i, the off-diagonal A tiles
//   C  chain: Q K^T tiles of chunk i + 1 -> M
//      prep:  the off-diagonal T tiles (one column chain per wave)
// Each chunk's rows are loaded one iteration before their LDS staging.
//
// Precision: fp32 operands enter the MFMAs as bf16 hi + lo with hi*hi + hi*lo + lo*hi (about 16 mantissa
// bits) where they feed the state (the state in K St, R, T, v_new in the state update, the inverse);
// bf16 inputs (k, q, v) enter exactly. Products that only feed the bf16 output (Q St, M v_new) take the
// bf16 rounding of their fp32 operand. Decays are e^x = 2^{x log2 e} on v_exp_f32 (G kept in log2 units).
// MFMA: v_mfma_f32_16x16x16_bf16 (A = row l % 16, k = 4 (l / 16) .. + 3; B = column l % 16, same k;
// the accumulator holds rows 4 (l / 16) .. + 3 of column l % 16, the B layout of the next product) and
// v_mfma_f32_16x16x32_bf16 for the K K^T / Q K^T tiles (k = 8 (l / 16) .. + 7).
#include <math.h>

#include "common.h"
#include "gdn_prefix.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int DK = 128;
constexpr int CH = 64;  // rows per chunk
constexpr int DS = 16;  // value columns per workgroup
constexpr int kNW = 8;
constexpr int kNT = kNW * kWave;
constexpr int TS = 68;  // bf16 row stride of T and M: 8-byte fragment reads of 16 rows hit distinct banks
constexpr int FS = 20;  // fp32 row stride of the 16 x 16 preparation tiles

__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}
__device__ __forceinline__ s16x4 as_s16(u32x2 v) { return __builtin_bit_cast(s16x4, v); }

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

// K / Q rows [CH][DK] bf16: 16-byte groups XOR-swizzled by the row
__device__ __forceinline__ int kq_off(int r, int grp) { return r * DK + ((grp ^ (r & 15)) << 3); }
__device__ __forceinline__ int kq_off4(int r, int d0) { return kq_off(r, d0 >> 3) + (d0 & 7); }  // d0 % 4 == 0
// K^T [DK][CH] bf16: 4-element groups XOR-swizzled so that both the staging writes (16 rows d = 8 g + e)
// and the fragment reads (16 rows d = 16 m + l % 16) of a wave quarter land on distinct groups
__device__ __forceinline__ int kt_off(int d, int s0) { return d * CH + (((s0 >> 2) ^ ((d ^ (d >> 3)) & 15)) << 2); }

struct Lds {
  // two buffers (chunk parity) of everything staged from HBM
  uint16_t K[2][CH * DK];
  uint16_t Q[2][CH * DK];
  uint16_t KT[2][DK * CH];
  uint16_t V[2][CH * DS];  // this workgroup's value columns
  float vec[2][5][CH];     // G log2(e), beta, e^G, e^{G_L - G}, e^{G_L} (every entry)
  uint16_t Th[CH * TS], Tl[CH * TS], Mh[CH * TS];
  u32x2 xRh[4][kWave], xRl[4][kWave];        // R row tiles hi / lo (B fragments)
  u32x2 xSh[8][kWave], xSl[8][kWave];        // state tiles hi / lo (B fragments)
  __align__(16) float Dd[4][16 * FS];        // inverses of the diagonal blocks, row-major fp32
  u32x2 Ao[6][2][kWave];                     // off-diagonal A tiles (1,0) (2,0) (2,1) (3,0) (3,1) (3,2) as
                                             // A fragments, hi and lo
};
static_assert(sizeof(Lds) <= 160 * 1024, "LDS plan exceeds 160 KiB");

// the rows of one chunk that a preparation wave stages: K and Q rows 16 pw + 4 (l / 16) + u (u = 0..3),
// columns 8 (l % 16) .. + 7; V row 16 pw + l / 4, columns 4 (l % 4) .. + 3; g and beta of row l
struct Raw {
  u32x4 k[4], q[4];
  u32x2 v;
  float g, be;
};

template <bool OUT>
__device__ __forceinline__ void load_raw(Raw& r, const PrefixArgs& a, int b, int h, int hk, int dv0, int c, int pw,
                                         int l) {
  const int t0 = c * CH;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int t = t0 + 16 * pw + 4 * (l / 16) + u;
    const bool ok = t < a.T;
    const int64_t off = ((int64_t)(b * a.T + (ok ? t : 0)) * a.Hk + hk) * DK + 8 * (l % 16);
    // rows past T read row 0 (in bounds) and are zeroed after the load: no branch around the loads
    const u32x4 kv = *reinterpret_cast<const u32x4*>(a.k + off);
    r.k[u] = ok ? kv : u32x4{0u, 0u, 0u, 0u};
    if (OUT) {
      const u32x4 qv = *reinterpret_cast<const u32x4*>(a.q + off);
      r.q[u] = ok ? qv : u32x4{0u, 0u, 0u, 0u};
    }
  }
  {
    const int t = t0 + 16 * pw + l / 4;
    const bool ok = t < a.T;
    const int64_t off = ((int64_t)(b * a.T + (ok ? t : 0)) * a.Hv + h) * a.Dv + dv0 + 4 * (l % 4);
    const u32x2 vv = *reinterpret_cast<const u32x2*>(a.v + off);
    r.v = ok ? vv : u32x2{0u, 0u};
  }
  {
    const int t = t0 + l;
    const bool ok = t < a.T;
    const int64_t gi = (int64_t)(b * a.T + (ok ? t : 0)) * a.Hv + h;
    const float gv = a.g[gi], bv = a.beta[gi];
    r.g = ok ? gv : 0.f;
    r.be = ok ? bv : 0.f;
  }
}

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
__device__ __forceinline__ f32x4 prod_ao(const Lds& sh, int idx, s16x4 yh, s16x4 yl, f32x4 c, int l) {
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
__device__ __forceinline__ void put_t(Lds& sh, int ti, int tj, f32x4 x, int l) {
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

__device__ __forceinline__ void lds_order() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
// workgroup barrier over LDS only: the preparation waves' global loads stay in flight across it
__device__ __forceinline__ void bar() {
  lds_order();
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <bool OUT>
struct Prefix {
  const PrefixArgs& a;
  Lds& sh;
  int b, h, hk, dv0, w, l, n;

  // ------------------------------------------------------------------ chain (waves 0-3), chunk i
  __device__ __forceinline__ void chain_a(int i, f32x4& qs) {
    const int kb = i & 1;
    f32x4 ks = {0.f, 0.f, 0.f, 0.f};
    qs = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = 16 * w + l % 16;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      const s16x4 sh_ = as_s16(sh.xSh[m][l]), sl_ = as_s16(sh.xSl[m][l]);
      const int o = kq_off4(r, 16 * m + 4 * (l / 16));
      const s16x4 ka = as_s16(*reinterpret_cast<const u32x2*>(&sh.K[kb][o]));
      ks = mma16(ka, sh_, ks);
      ks = mma16(ka, sl_, ks);
      if (OUT) {
        const s16x4 qa = as_s16(*reinterpret_cast<const u32x2*>(&sh.Q[kb][o]));
        qs = mma16(qa, sh_, qs);  // Q St feeds only the bf16 output: the state's hi part
      }
    }
    f32x4 R;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = 16 * w + 4 * (l / 16) + e;
      R[e] = sh.vec[kb][1][t] * (bf2f(sh.V[kb][t * DS + l % 16]) - sh.vec[kb][2][t] * ks[e]);
    }
    s16x4 rh, rl;
    split4(R, rh, rl);
    sh.xRh[w][l] = __builtin_bit_cast(u32x2, rh);
    sh.xRl[w][l] = __builtin_bit_cast(u32x2, rl);
  }

  __device__ __forceinline__ void chain_b(int i, f32x4 qs, f32x4 (&st)[2]) {
    const int kb = i & 1;
    s16x4 rh[4], rl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      rh[kt] = as_s16(sh.xRh[kt][l]);
      rl[kt] = as_s16(sh.xRl[kt][l]);
    }
    f32x4 vn[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt <= it; ++kt) {
        const int o = (16 * it + l % 16) * TS + 16 * kt + 4 * (l / 16);
        const s16x4 th = as_s16(*reinterpret_cast<const u32x2*>(&sh.Th[o]));
        const s16x4 tl = as_s16(*reinterpret_cast<const u32x2*>(&sh.Tl[o]));
        c = mm3(th, tl, rh[kt], rl[kt], c);
      }
      vn[it] = c;
    }
    if (OUT) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        if (kt <= w) {  // M v_new feeds only the bf16 output: hi parts
          const s16x4 mh = as_s16(*reinterpret_cast<const u32x2*>(&sh.Mh[(16 * w + l % 16) * TS + 16 * kt + 4 * (l / 16)]));
          acc = mma16(mh, hi4(vn[kt]), acc);
        }
      }
      const int64_t vrow = (int64_t)a.Hv * a.Dv;
      uint16_t* ob = a.out + (int64_t)b * a.T * vrow + (int64_t)h * a.Dv + dv0 + l % 16;
      uint16_t ov[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ov[e] = f2bf(a.scale * (sh.vec[kb][2][16 * w + 4 * (l / 16) + e] * qs[e] + acc[e]));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tg = i * CH + 16 * w + 4 * (l / 16) + e;
        if (tg < a.T) ob[(int64_t)tg * vrow] = ov[e];
      }
    }
    // state: St' = e^{G_L} St + K^T diag(e^{G_L - G}) v_new on this wave's Dk tiles 2w, 2w+1
    s16x4 ph[4], pl[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      f32x4 vp;
#pragma unroll
      for (int e = 0; e < 4; ++e) vp[e] = vn[kt][e] * sh.vec[kb][3][16 * kt + 4 * (l / 16) + e];
      split4(vp, ph[kt], pl[kt]);
    }
    const float eL = sh.vec[kb][4][0];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = 2 * w + j;
      f32x4 s = st[j] * eL;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const s16x4 ka =
            as_s16(*reinterpret_cast<const u32x2*>(&sh.KT[kb][kt_off(16 * m + l % 16, 16 * kt + 4 * (l / 16))]));
        s = mma16(ka, ph[kt], s);
        s = mma16(ka, pl[kt], s);
      }
      st[j] = s;
      s16x4 hh, ll;
      split4(s, hh, ll);
      sh.xSh[m][l] = __builtin_bit_cast(u32x2, hh);
      sh.xSl[m][l] = __builtin_bit_cast(u32x2, ll);
    }
  }

  // Q K^T tiles of chunk c (lower triangle, 10 tiles; wave w takes tiles w, w + 4, w + 8) -> M (bf16)
  __device__ __forceinline__ void chain_c(int c) {
    const int kb = c & 1;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int idx = w + 4 * j;
      if (idx < 10) {
        const int ti = idx < 1 ? 0 : idx < 3 ? 1 : idx < 6 ? 2 : 3;
        const int tj = idx - ti * (ti + 1) / 2;
        const f32x4 cq = xk_tile(sh.Q[kb], sh.K[kb], ti, tj, l);
        const int s = 16 * tj + l % 16;
        const float Gs = sh.vec[kb][0][s];
#pragma unroll
        for (int e = 0; e < 4; ++e) {  // branch-free: the decay is clamped to <= 0 where it is masked out
          const int t = 16 * ti + 4 * (l / 16) + e;
          const float x = cq[e] * ex2(fminf(sh.vec[kb][0][t] - Gs, 0.f));
          sh.Mh[t * TS + s] = f2bf(s <= t ? x : 0.f);
        }
      }
    }
  }

  // ------------------------------------------------------------------ preparation (waves 4-7), chunk c
  __device__ __forceinline__ void prep_a(int c, Raw& cur) {
    const int kb = c & 1, pw = w - 4;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int o = kq_off(16 * pw + 4 * (l / 16) + u, l % 16);
      *reinterpret_cast<u32x4*>(&sh.K[kb][o]) = cur.k[u];
      if (OUT) *reinterpret_cast<u32x4*>(&sh.Q[kb][o]) = cur.q[u];
    }
    // K^T: the lane holds K[16 pw + 4 (l / 16) + u][8 (l % 16) + e], u = 0..3
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint32_t x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = (cur.k[u][e >> 1] >> (16 * (e & 1))) & 0xffffu;
      *reinterpret_cast<u32x2*>(&sh.KT[kb][kt_off(8 * (l % 16) + e, 16 * pw + 4 * (l / 16))]) =
          u32x2{x[0] | (x[1] << 16), x[2] | (x[3] << 16)};
    }
    *reinterpret_cast<u32x2*>(&sh.V[kb][(16 * pw + l / 4) * DS + 4 * (l % 4)]) = cur.v;
    if (pw == 0) {
      float G = cur.g;
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const float o = __shfl_up(G, off, kWave);
        if (l >= off) G += o;
      }
      G *= kLog2e;
      const float GL = __shfl(G, kWave - 1, kWave);
      sh.vec[kb][0][l] = G;
      sh.vec[kb][1][l] = cur.be;
      sh.vec[kb][2][l] = ex2(G);
      sh.vec[kb][3][l] = ex2(GL - G);
      sh.vec[kb][4][l] = ex2(GL);
    }
    // the next chunk's rows: in flight until the next iteration's phase A
    if (c + 1 < n) load_raw<OUT>(cur, a, b, h, hk, dv0, c + 1, pw, l);
  }

  __device__ __forceinline__ void prep_b(int c) {
    const int kb = c & 1, pw = w - 4;
    const uint16_t* Kc = sh.K[kb];
    const float* G2 = sh.vec[kb][0];
    const float* be = sh.vec[kb][1];
    const int r = l % 16, q4 = 4 * (l / 16);
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    // Diagonal block pw: N = -A_pp in both operand layouts from the one (symmetric) K K^T tile, then
    // D = (I - N)^{-1} = (I + N)(I + N^2)(I + N^4)(I + N^8) (N is strictly lower triangular, N^16 = 0).
    // The accumulator layout of X^T is the A layout of X, and the factors commute, so every product
    // takes both operands from registers.
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
    // Off-diagonal A tiles (wave 4: (1,0) (2,0); 5: (2,1) (3,0); 6: (3,1); 7: (3,2)), each from the
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

  __device__ __forceinline__ void prep_c() {
    const int pw = w - 4;
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
      const f32x4 y3 =
          prod_ao(sh, 5, h20, l20, prod_ao(sh, 4, h10, l10, prod_ao(sh, 3, dh, dl, z, l), l), l);
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

  // one preparation iteration: chunk c = i + 1 (< n) from register set cur
  __device__ __forceinline__ void prep_step(int i, Raw& cur) {
    const int c = i + 1;
    if (c < n) prep_a(c, cur);
    bar();
    if (c < n) prep_b(c);
    bar();
    if (c < n) prep_c();
    bar();
  }
};

template <bool OUT>
__global__ __launch_bounds__(kNT) void gdr_prefix_kernel(PrefixArgs a) {
  __shared__ __align__(16) Lds sh;
  const int slices = a.Dv / DS;
  int idx = xcd_major(blockIdx.x, gridDim.x);  // a head's value slices (same K / Q rows) on one XCD
  const int sl = idx % slices;
  idx /= slices;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave), l = threadIdx.x % kWave;
  Prefix<OUT> p{a, sh, idx / a.Hv, idx % a.Hv, (idx % a.Hv) / (a.Hv / a.Hk), sl * DS, w, l, a.nchunks};
  // The two roles run separate loops with the same barrier sequence: n + 1 iterations of three phases
  // (iteration i: chain on chunk i when i >= 0, preparation of chunk i + 1 when i + 1 < n).
  if (w < 4) {
    f32x4 st[2];
    const int64_t soff = (((int64_t)p.b * a.Hv + p.h) * a.Dv + p.dv0 + l % 16) * DK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int m = 2 * w + j;
      st[j] = *reinterpret_cast<const f32x4*>(a.state_in + soff + 16 * m + 4 * (l / 16));
      s16x4 hh, ll;
      split4(st[j], hh, ll);
      sh.xSh[m][l] = __builtin_bit_cast(u32x2, hh);
      sh.xSl[m][l] = __builtin_bit_cast(u32x2, ll);
    }
    for (int i = -1; i < p.n; ++i) {
      f32x4 qs = {0.f, 0.f, 0.f, 0.f};
      if (i >= 0) p.chain_a(i, qs);
      bar();
      if (i >= 0) p.chain_b(i, qs, st);
      bar();
      if (OUT && i + 1 < p.n) p.chain_c(i + 1);
      bar();
    }
    if (a.state_out) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
        *reinterpret_cast<f32x4*>(a.state_out + soff + 16 * (2 * w + j) + 4 * (l / 16)) = st[j];
    }
  } else {
    // chunk c's rows are loaded one iteration ahead of their staging
    Raw r;
    load_raw<OUT>(r, a, p.b, p.h, p.hk, p.dv0, 0, w - 4, l);
    for (int i = -1; i < p.n; ++i) p.prep_step(i, r);
  }
}

}  // namespace

bool gdr_prefix_supported(int64_t B, int64_t T, int64_t Hv, int64_t Dk, int64_t Dv) {
  // one workgroup per CU at most: the kernel is latency-bound per chunk, and a grid of several rounds
  // runs its chunk chains one round after the other (larger batches take the prep + scan kernels)
  return T > CH && Dk == DK && Dv % DS == 0 && B * Hv * (Dv / DS) <= 256;
}

int gdr_prefix_launch(const PrefixArgs& a, int64_t B, hipStream_t stream) {
  const dim3 grid((unsigned)(B * a.Hv * (a.Dv / DS)));
  if (a.out) hipLaunchKernelGGL(gdr_prefix_kernel<true>, grid, dim3(kNT), 0, stream, a);
  else hipLaunchKernelGGL(gdr_prefix_kernel<false>, grid, dim3(kNT), 0, stream, a);
  return launch_status("gdr_chunk/prefix");
}

}  // namespace trida
