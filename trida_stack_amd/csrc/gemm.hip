// Weight-streaming bf16 GEMM for the decode-step projections: Y[M, N] = X[M, K] W[N, K]^T with M <= 48
// (a canvas of <= 48 rows), fp32 accumulation. At these M every projection is bound by the weight stream
// (N * K * 2 bytes read once), so the kernel is built around that stream:
//   - the weights are stored once more in a pre-shuffled layout (trida_wsgemm_shuffle): tile t of 16
//     rows, k-step s of 32 columns, lane l = 16 g + r holds W[16 t + r][32 s + 8 g .. + 8] as 16 bytes, the
//     A operand of v_mfma_f32_16x16x32_bf16 as it lands in a register. A wave's walk over one tile is
//     then one contiguous run of memory;
//   - X is stationary: wave w of a workgroup owns KWS consecutive k-steps and loads its slice of X (the
//     B operand, tokens as columns) into registers once; it then streams the weights of the workgroup's
//     T tiles over that K slice with D k-steps of loads in flight (a register ring whose loads are pinned
//     in issue order by sched_barrier, so the compiler neither sinks them nor drains the ring);
//   - each wave parks its partial 16 x 16*MT tile of every finished tile in an LDS slot and streams on;
//     when the slots are full or the tiles done, the workgroup meets once and all its threads sum the
//     parked tiles in wave order and run the epilogue. A plan's T tiles fit in the slots, so the weight
//     stream never waits on another wave (longer plans flush every NSLOT tiles);
//   - X rows past M are not loaded (lanes masked), so a 33-row canvas moves 2 KB + 64 B of X per k-step;
//   - X may come in fragment order (Xf[s][mt][lane], lane 16 g + r holding X[16 mt + r][32 s + 8 g .. + 8],
//     mt stride kWsFragMT whatever M is): every X load of a wave is then 1 KB of consecutive bytes, whole
//     cache lines, where row-major X gives each load 16 rows x 64 B, half a line per row (the whole slice of
//     a 33-row canvas: 2.4 instead of 4.6 us per workgroup). The producers of the decode-step activations
//     (trida_residual_parts_frag, trida_gated_rmsnorm_frag, this kernel's own epilogues) write that order;
//   - K beyond NW * KWS steps is split over kg workgroup groups that write fp32 partial planes
//     [kg][M][N]; trida_add_rmsnorm_parts (norms.hip) sums them in plane order;
//   - per-head row scales (trida_wsgemm_headnorm, partial planes): when a wave's K slice is one head of X
//     (KWS * 32 = the head width), its partial sums of a row are multiplied by rsqrt(mean of the row's head
//     squares + eps) from per-piece sums of squares before they are parked: the gated RMSNorm of a GDN
//     layer applied to X = o * w * silu(z) after the product instead of before it.
// Epilogues: bf16 store, fp32 partials, SwiGLU (silu(gate) * up) over weights whose tiles interleave 8
// gate rows with the matching 8 up rows, or argmax: the LM head of a greedy verify reduces each row of its
// bf16 logits to the workgroup's (max, first index) in registers while the weights stream, and writes one
// pair per row and workgroup (optionally the logits too), so acceptance never reads the logits again; with
// the softmax denominator too (argmax + confidence, a denoise pass's readout): sum exp(x - max) over the
// workgroup's columns, relative to its max. The plan (NW, KWS, T, kg) depends on N, K and the epilogue only:
// a row of Y is bitwise the same whether X holds 1 row or 48.
#include <algorithm>

#include "common.h"

namespace trida {
namespace {

constexpr int kCUs = 256;  // MI355X (gfx950): workgroups of a plan <= one per CU, see plan_for()
constexpr int kMaxM = 48;

enum Epilogue { kStore = 0, kParts = 1, kSilu = 2, kArgmax = 3, kArgmaxConf = 4 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ bf16x8 as_bf(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }
__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }

struct WsArgs {
  const uint16_t* X;
  const u32x4* Wp;
  void* out;
  int64_t x_st, o_st;
  int M, N, K, T;
  // RMSNorm (NORM kernels): X is the raw residual stream and the weights were shuffled with the norm weight
  // folded into their columns, so row m of the result is inv_m * (X W'^T)[m], inv_m = rsqrt(sum_c ss[m][c] /
  // K + eps) over the ss_chunks(K) per-chunk sums of squares, applied in the epilogue
  const float* ss;
  float eps;
  int xf;  // X in fragment order (x_st unused)
  int of;  // bf16 output (store / SwiGLU epilogues) in fragment order for the next GEMM (o_st unused)
  float* pval;  // argmax epilogue: [M][gridDim.x] best value of each row within each workgroup's columns
  int* pidx;    // and its column (first on ties, NaN first)
  float* psum;  // argmax + confidence: [M][gridDim.x] sum exp(x - pval) over the workgroup's columns
  // per-head row scales: [M][h_heads][head width / 8] sums of squares of X's 8-column pieces, or null
  const float* hss;
  int h_heads;
  float h_eps;
};


// chunks of the per-row sums of squares that trida_residual_parts writes: 256 elements each
__host__ __device__ constexpr int ss_chunks(int dim) { return (dim + 255) / 256; }
constexpr int kMaxSsChunks = 10;  // K <= 2560: every whole-K plan (<= 80 k-steps)

// LDS slots of partial tiles: as many as fit in 144 KiB, at most 8
template <int NW, int MT>
constexpr int nslot() {
  return (147456 / (NW * MT * 1024)) < 8 ? (147456 / (NW * MT * 1024)) : 8;
}

template <int NW, int KWS, int D, int MT, int EPI, bool NORM>
__global__ __launch_bounds__(NW* kWave) void wsgemm_kernel(WsArgs a) {
  static_assert(KWS % D == 0 || D % KWS == 0, "the ring and the K slice must tile the unrolled loop");
  constexpr bool AMAX = EPI == kArgmax || EPI == kArgmaxConf, CONF = EPI == kArgmaxConf;
  constexpr int NSLOT = nslot<NW, MT>();
  static_assert(NSLOT >= 2, "LDS slots");
  __shared__ f32x4 red[NSLOT][NW][MT][kWave];
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int tiles = a.N / 16, nsteps = a.K / 32;
  const int t0 = blockIdx.x * a.T, nt = min(tiles, t0 + a.T) - t0;
  const int s_base = (blockIdx.y * NW + wave) * KWS;
  const int my_steps = max(0, min(KWS, nsteps - s_base));  // k-steps of this wave inside K

  // weight stream: unit u = (tile t0 + u / KWS, k-step s_base + u % KWS); loads past the last unit
  // re-read it and steps past K read the last step (in bounds; their X is zero)
  const int nu = nt * KWS;
  auto wptr = [&](int u) {
    u = min(u, nu - 1);
    const int t = t0 + u / KWS, s = min(s_base + u % KWS, nsteps - 1);
    return a.Wp + ((int64_t)t * nsteps + s) * kWave + l;
  };
  u32x4 wv[D];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    wv[j] = *wptr(j);
    __builtin_amdgcn_sched_barrier(0);
  }
  // X slice (issued after the first weight loads, so their latency overlaps): lanes of tokens past M
  // load nothing (their columns are never stored); steps past K are zero
  u32x4 xs[KWS][MT];
  if (a.xf) {
    const u32x4* xb = reinterpret_cast<const u32x4*>(a.X) + l;
#pragma unroll
    for (int j = 0; j < KWS; ++j) {
      const int s = min(s_base + j, nsteps - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        xs[j][mt] = u32x4{0u, 0u, 0u, 0u};
        if (mt * 16 + (l % 16) < a.M && j < my_steps) xs[j][mt] = xb[((int64_t)s * kWsFragMT + mt) * kWave];
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < KWS; ++j) {
      const int s = min(s_base + j, nsteps - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + (l % 16);
        xs[j][mt] = u32x4{0u, 0u, 0u, 0u};
        if (m < a.M && j < my_steps)
          xs[j][mt] = *reinterpret_cast<const u32x4*>(a.X + (int64_t)m * a.x_st + s * 32 + (l / 16) * 8);
      }
    }
  }
  // per-head row scales of this wave's head (K slice = one head): lane group l / 16 sums a quarter of the
  // row's piece sums, two xor exchanges the rest
  float hinv[MT];
  const bool hscale = EPI == kParts && a.hss;  // the partial-plane kernels only
  if (hscale) {
    constexpr int P = KWS * 32 / 8;  // 8-column pieces of the head
    const int head = min((int)blockIdx.y * NW + wave, a.h_heads - 1);
    float hp[MT][P / 4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float* src = a.hss + ((int64_t)min(mt * 16 + (l % 16), a.M - 1) * a.h_heads + head) * P + (l / 16) * (P / 4);
#pragma unroll
      for (int j = 0; j < P / 4; ++j) hp[mt][j] = src[j];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      float q = 0.f;
#pragma unroll
      for (int j = 0; j < P / 4; ++j) q += hp[mt][j];
      q += __shfl_xor(q, 16, kWave);
      q += __shfl_xor(q, 32, kWave);
      hinv[mt] = rsqrtf(q / (float)(KWS * 32) + a.h_eps);
    }
  }
  // Wait for the prologue's loads here: the first MFMA needs the last of them anyway (X was issued after
  // the ring), and a known-empty queue lets the compiler count the ring's loads exactly in the loop (the
  // masked X loads would otherwise make it drain the ring at every pass). vmcnt(0) only (gfx9 encoding:
  // expcnt and lgkmcnt at their maximum).
  __builtin_amdgcn_s_waitcnt(0x0F70);
  // RMSNorm scale of each token, for the epilogue: wave 0 sums the token's chunk sums of squares in chunk
  // order (whole-K plans have K <= 2560, i.e. <= 10 chunks: unrolled, unconditional loads); the first flush's
  // barrier publishes them
  __shared__ float inv_s[MT * 16];
  if (NORM && threadIdx.x < MT * 16) {
    const int C = ss_chunks(a.K);
    const int m = min((int)threadIdx.x, a.M - 1);
    float v[kMaxSsChunks];
#pragma unroll
    for (int c = 0; c < kMaxSsChunks; ++c) v[c] = a.ss[(int64_t)m * C + min(c, C - 1)];
    float sum = 0.f;
#pragma unroll
    for (int c = 0; c < kMaxSsChunks; ++c) sum += c < C ? v[c] : 0.f;
    inv_s[threadIdx.x] = rsqrtf(sum / (float)a.K + a.eps);
  }

  // argmax epilogue: this thread's running (value, column) of rows mm * 16 + l % 16, over the columns its
  // flush items covered (the lanes l, l ^ 16, l ^ 32, l ^ 48 and the waves are merged at the end)
  float hv[MT];
  int hi[MT];
  float sm[MT], ss[MT];  // CONF: the running (max, sum exp(x - max)) of the same rows and columns
#pragma unroll
  for (int mm = 0; mm < MT; ++mm) {
    hv[mm] = -INFINITY;
    hi[mm] = INT32_MAX;
    sm[mm] = -INFINITY;
    ss[mm] = 0.f;
  }
  // 4 consecutive bf16 outputs (n % 4 == 0) of row m: row-major, or in fragment order for the next GEMM
  auto out_at = [&](int m, int n) -> u32x2* {
    uint16_t* o = static_cast<uint16_t*>(a.out);
    return reinterpret_cast<u32x2*>(a.of ? o + ws_frag_off(m, n) : o + (int64_t)m * a.o_st + n);
  };
  // tiles [first, last] are parked in their slots: meet, sum the NW partials of each in wave order, run the
  // epilogue (64 * NW threads over the parked tiles' outputs)
  auto flush = [&](int first, int last) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // LDS only: the weight loads stay in flight
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    constexpr int per_tile = EPI == kSilu ? MT * 32 : MT * kWave;
    const int items = (last - first + 1) * per_tile;
    for (int it = threadIdx.x; it < items; it += NW * kWave) {
      const int tl = first + it / per_tile, q = it % per_tile;
      const int slot = tl % NSLOT, tile = t0 + tl;
      if (EPI == kSilu) {
        // lanes 0..31 of a C tile hold rows 0..7 (gate), lanes 32..63 rows 8..15 (the matching up)
        const int mt = q / 32, ln = q % 32;
        f32x4 g = red[slot][0][mt][ln], up = red[slot][0][mt][ln + 32];
#pragma unroll
        for (int w = 1; w < NW; ++w) {
          g += red[slot][w][mt][ln];
          up += red[slot][w][mt][ln + 32];
        }
        const int m = mt * 16 + (ln % 16);
        if (NORM) {
          const float inv = inv_s[m];
          g *= inv;
          up *= inv;
        }
        if (m < a.M) {
          const int f = tile * 8 + (ln / 16) * 4;
          const float y0 = silu(bf2f(f2bf(g.x))) * bf2f(f2bf(up.x));
          const float y1 = silu(bf2f(f2bf(g.y))) * bf2f(f2bf(up.y));
          const float y2 = silu(bf2f(f2bf(g.z))) * bf2f(f2bf(up.z));
          const float y3 = silu(bf2f(f2bf(g.w))) * bf2f(f2bf(up.w));
          u32x2 packed;
          packed.x = f2bf2(y0, y1);
          packed.y = f2bf2(y2, y3);
          *out_at(m, f) = packed;
        }
      } else if (AMAX) {
        // mt is uniform over a wave (its 64 items are consecutive and a tile's items come in whole waves)
        const int mt = q / kWave, ln = q % kWave;
        f32x4 sum = red[slot][0][mt][ln];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[slot][w][mt][ln];
        const int m = mt * 16 + (ln % 16);
        const int n = tile * 16 + (ln / 16) * 4;
        if (NORM) sum *= inv_s[m];
        // the bf16 logits, as the store epilogue writes them; the argmax compares their fp32 widening
        const uint32_t p0 = f2bf2(sum.x, sum.y), p1 = f2bf2(sum.z, sum.w);
        if (a.out && m < a.M) *out_at(m, n) = u32x2{p0, p1};
        const float v[4] = {__uint_as_float(p0 << 16), __uint_as_float(p0 & 0xffff0000u), __uint_as_float(p1 << 16),
                            __uint_as_float(p1 & 0xffff0000u)};
        float bv = v[0];
        int bi = n;
#pragma unroll
        for (int e = 1; e < 4; ++e)
          if (argmax_better(v[e], n + e, bv, bi)) {
            bv = v[e];
            bi = n + e;
          }
#pragma unroll
        for (int mm = 0; mm < MT; ++mm) {
          if (mm == mt && argmax_better(bv, bi, hv[mm], hi[mm])) {
            hv[mm] = bv;
            hi[mm] = bi;
          }
          if (CONF && mm == mt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc_exp(v[e], true, sm[mm], ss[mm]);
          }
        }
      } else {
        const int mt = q / kWave, ln = q % kWave;
        f32x4 sum = red[slot][0][mt][ln];
#pragma unroll
        for (int w = 1; w < NW; ++w) sum += red[slot][w][mt][ln];
        const int m = mt * 16 + (ln % 16);
        const int n = tile * 16 + (ln / 16) * 4;
        if (NORM) sum *= inv_s[m];
        if (m < a.M) {
          if (EPI == kStore) {
            u32x2 packed;
            packed.x = f2bf2(sum.x, sum.y);
            packed.y = f2bf2(sum.z, sum.w);
            *out_at(m, n) = packed;
          } else {
            *reinterpret_cast<f32x4*>(static_cast<float*>(a.out) + ((int64_t)blockIdx.y * a.M + m) * a.N + n) = sum;
          }
        }
      }
    }
    if (last + 1 < nt) {  // the slots are rewritten: every thread has finished reading them
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }
  };

  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  constexpr int U = KWS > D ? KWS : D;  // units per unrolled pass: ring slot and X step are static
  for (int u0 = 0; u0 < nu; u0 += U) {
#pragma unroll
    for (int jj = 0; jj < U; ++jj) {
      const int u = u0 + jj;
      const int j = jj % KWS, r = jj % D;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(wv[r]), as_bf(xs[j][mt]), acc[mt], 0, 0, 0);
      wv[r] = *wptr(u + D);
      __builtin_amdgcn_sched_barrier(0);
      const int tl = u / KWS;
      if (j == KWS - 1 && tl < nt) {  // this wave's part of tile tl is complete (uniform condition)
        const int slot = tl % NSLOT;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          red[slot][wave][mt][l] = hscale ? acc[mt] * hinv[mt] : acc[mt];
          acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        if (slot == NSLOT - 1 || tl == nt - 1) flush(tl - slot, tl);
      }
    }
  }
  if constexpr (AMAX) {
    // merge the four lanes of each row, then the waves in order; one (value, column) per row
    __shared__ float s_bv[NW][MT * 16];
    __shared__ int s_bi[NW][MT * 16];
    __shared__ float s_sm[CONF ? NW : 1][MT * 16], s_ss[CONF ? NW : 1][MT * 16];
#pragma unroll
    for (int mm = 0; mm < MT; ++mm) {
#pragma unroll
      for (int off = 16; off < kWave; off <<= 1) {
        const float ov = __shfl_xor(hv[mm], off, kWave);
        const int oi = __shfl_xor(hi[mm], off, kWave);
        if (argmax_better(ov, oi, hv[mm], hi[mm])) {
          hv[mm] = ov;
          hi[mm] = oi;
        }
        if (CONF) {
          const float om = __shfl_xor(sm[mm], off, kWave), os = __shfl_xor(ss[mm], off, kWave);
          merge_exp(sm[mm], ss[mm], om, os);
        }
      }
      if (l < 16) {
        s_bv[wave][mm * 16 + l] = hv[mm];
        s_bi[wave][mm * 16 + l] = hi[mm];
        if (CONF) {
          s_sm[wave][mm * 16 + l] = sm[mm];
          s_ss[wave][mm * 16 + l] = ss[mm];
        }
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < a.M) {
      const int m = threadIdx.x;
      float v = s_bv[0][m];
      int i = s_bi[0][m];
#pragma unroll
      for (int w = 1; w < NW; ++w)
        if (argmax_better(s_bv[w][m], s_bi[w][m], v, i)) {
          v = s_bv[w][m];
          i = s_bi[w][m];
        }
      a.pval[(int64_t)m * gridDim.x + blockIdx.x] = v;
      a.pidx[(int64_t)m * gridDim.x + blockIdx.x] = i;
      if (CONF) {
        float mx = s_sm[0][m], sum = s_ss[0][m];
#pragma unroll
        for (int w = 1; w < NW; ++w) merge_exp(mx, sum, s_sm[w][m], s_ss[w][m]);
        // relative to the workgroup's argmax value (the row max is found among these)
        a.psum[(int64_t)m * gridDim.x + blockIdx.x] = (mx == -INFINITY || v != v) ? 0.f : sum * __expf(mx - v);
      }
    }
  }
}

// pre-shuffle: one thread per 16-byte piece of Wp, in Wp order
__global__ __launch_bounds__(256) void shuffle_kernel(const uint16_t* W, int64_t ld, int N, int K, int pair,
                                                      const uint16_t* col_scale, int zero_centred, u32x4* Wp) {
  const int64_t nsteps = K / 32, total = (int64_t)(N / 16) * nsteps * kWave;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int lane = (int)(i % kWave);
  const int64_t rest = i / kWave;
  const int s = (int)(rest % nsteps), t = (int)(rest / nsteps);
  const int r = lane % 16, g = lane / 16;
  const int row = pair ? (r < 8 ? 8 * t + r : N / 2 + 8 * t + (r - 8)) : 16 * t + r;
  const int k0 = s * 32 + g * 8;
  u32x4 v = *reinterpret_cast<const u32x4*>(W + (int64_t)row * ld + k0);
  if (col_scale) {  // W'[row][k] = bf16(W[row][k] * (1 + c[k])) (zero_centred) or bf16(W[row][k] * c[k])
    const u32x4 cv = *reinterpret_cast<const u32x4*>(col_scale + k0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float c0 = bf2f((uint16_t)(cv[q] & 0xffff)), c1 = bf2f((uint16_t)(cv[q] >> 16));
      if (zero_centred) {
        c0 = 1.f + c0;
        c1 = 1.f + c1;
      }
      v[q] = f2bf2(bf2f((uint16_t)(v[q] & 0xffff)) * c0, bf2f((uint16_t)(v[q] >> 16)) * c1);
    }
  }
  Wp[i] = v;
}

// ---------------------------------------------------------------- plans
struct Cfg {
  int nw, kws;
  bool head_only;  // only for per-head-scaled products whose heads are kws k-steps wide
};
// 16-wave workgroups measured 10-15% slower; {8, 2} serves heads of 64 columns (partial planes only)
constexpr Cfg kCfgs[] = {{8, 10, false}, {8, 5, false}, {8, 4, false}, {8, 2, true}};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

struct Plan {
  int cfg, T, kg;
};

// Deterministic plan from (N, K, epilogue): for each kernel shape, the fewest tiles per workgroup that keep
// the grid within one workgroup per CU (a CU that had to run two would finish last), then the lowest cost
// in units of one weight k-step of a workgroup (~0.05 us measured at 33 rows): the k-steps per workgroup,
// + 4 per k-step of X slice (its load precedes the stream, ~0.2 us each), + 6 per extra partial plane
// (read again by its consumer: ~0.3 us per plane at 33 rows). Bf16 and SwiGLU epilogues need the whole K
// in one workgroup (kg == 1); ties go to the thinner X slice.
// kws > 0: only the configuration whose waves take kws k-steps each (a head per wave).
Plan plan_for(int64_t N, int64_t K, int epi, int kws = 0) {
  const int64_t tiles = N / 16, nsteps = K / 32;
  Plan best{-1, 0, 0};
  int64_t best_cost = INT64_MAX;
  for (int c = 0; c < kNumCfgs; ++c) {
    if (kws > 0 ? kCfgs[c].kws != kws : kCfgs[c].head_only) continue;
    const int64_t per = (int64_t)kCfgs[c].nw * kCfgs[c].kws;
    const int64_t kg = cdiv(nsteps, per);
    if (epi != kParts && kg != 1) continue;
    if (kg > 64) continue;
    const int64_t T = std::max<int64_t>(1, cdiv(tiles * kg, kCUs));
    const int64_t work = T * std::min(per, nsteps);
    const int64_t cost = work + 4 * kCfgs[c].kws + 6 * (kg - 1);
    if (cost < best_cost || (cost == best_cost && kCfgs[c].kws < kCfgs[best.cfg].kws)) {
      best_cost = cost;
      best = {c, (int)T, (int)kg};
    }
  }
  return best;
}

template <int NW, int KWS, int D, int MT, int EPI, bool NORM>
void launch(const WsArgs& a, int kg, hipStream_t st) {
  const dim3 grid((unsigned)cdiv(a.N / 16, a.T), (unsigned)kg);
  hipLaunchKernelGGL((wsgemm_kernel<NW, KWS, D, MT, EPI, NORM>), grid, dim3(NW * kWave), 0, st, a);
}
template <int NW, int KWS, int D, int EPI, bool NORM>
void launch_mt(const WsArgs& a, int kg, hipStream_t st) {
  switch ((a.M + 15) / 16) {
    case 1: launch<NW, KWS, D, 1, EPI, NORM>(a, kg, st); break;
    case 2: launch<NW, KWS, D, 2, EPI, NORM>(a, kg, st); break;
    default: launch<NW, KWS, D, 3, EPI, NORM>(a, kg, st); break;
  }
}
template <int EPI, bool NORM>
void launch_cfg(const WsArgs& a, const Plan& p, hipStream_t st) {
  switch (p.cfg) {
    case 0: launch_mt<8, 10, 10, EPI, NORM>(a, p.kg, st); break;
    case 1: launch_mt<8, 5, 10, EPI, NORM>(a, p.kg, st); break;
    case 2: launch_mt<8, 4, 8, EPI, NORM>(a, p.kg, st); break;
    default:
      if constexpr (EPI == kParts && !NORM) launch_mt<8, 2, 10, EPI, NORM>(a, p.kg, st);
      break;
  }
}

// residual add of split-K partial planes (grid rows x ss_chunks(dim), one wave per 256-element chunk):
// h = bf16(h + bf16(sum_s parts[s][row])) (planes summed in order; n_parts = 0 leaves h as it is), and
// ss[row][chunk] = the chunk's sum of h^2, which the RMSNorm prologue of the next GEMM reads; hf (rows <= 48,
// or null): h once more in fragment order, the next GEMM's X
__global__ __launch_bounds__(kWave) void residual_kernel(uint16_t* h, int64_t h_st, const float* parts, int n_parts,
                                                         int64_t plane_st, int dim, float* ss, uint16_t* hf) {
  const int64_t row = blockIdx.x;
  const int c = blockIdx.y, l = threadIdx.x;
  const int e = c * 256 + l * 4;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (e < dim) {
    uint16_t* hp = h + row * h_st + e;
    if (n_parts > 0) {
      // every plane's load issued first (8 loads; planes past n_parts re-read the last one, in bounds, and
      // are dropped), then h; branch-free; the sum stays in plane order
      const float* pp = parts + row * dim + e;
      f32x4 pv[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) pv[s] = *reinterpret_cast<const f32x4*>(pp + min(s, n_parts - 1) * plane_st);
      const u32x2 hv = *reinterpret_cast<const u32x2*>(hp);
      f32x4 acc = pv[0];
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 1; s < 8; ++s) acc += s < n_parts ? pv[s] : zero;
      for (int s = 8; s < n_parts; ++s) acc += *reinterpret_cast<const f32x4*>(pp + s * plane_st);
      // the residual stream is bf16
      v[0] = bf2f(f2bf(bf2f((uint16_t)(hv.x & 0xffff)) + bf2f(f2bf(acc.x))));
      v[1] = bf2f(f2bf(bf2f((uint16_t)(hv.x >> 16)) + bf2f(f2bf(acc.y))));
      v[2] = bf2f(f2bf(bf2f((uint16_t)(hv.y & 0xffff)) + bf2f(f2bf(acc.z))));
      v[3] = bf2f(f2bf(bf2f((uint16_t)(hv.y >> 16)) + bf2f(f2bf(acc.w))));
      *reinterpret_cast<u32x2*>(hp) = u32x2{f2bf2(v[0], v[1]), f2bf2(v[2], v[3])};
    } else {
      const u32x2 hv = *reinterpret_cast<const u32x2*>(hp);
      v[0] = bf2f((uint16_t)(hv.x & 0xffff));
      v[1] = bf2f((uint16_t)(hv.x >> 16));
      v[2] = bf2f((uint16_t)(hv.y & 0xffff));
      v[3] = bf2f((uint16_t)(hv.y >> 16));
    }
    if (hf) *reinterpret_cast<u32x2*>(hf + ws_frag_off((int)row, e)) = u32x2{f2bf2(v[0], v[1]), f2bf2(v[2], v[3])};
  }
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) q = fmaf(v[i], v[i], q);
  q = wave_sum(q);
  if (l == 0) ss[row * ss_chunks(dim) + c] = q;
}

// row-major X [M, K] to fragment order: one thread per 16-byte piece
__global__ __launch_bounds__(256) void frag_kernel(const uint16_t* X, int64_t x_st, int M, int K, uint16_t* Xf) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * (K / 8)) return;
  const int m = (int)(i / (K / 8)), k = (int)(i % (K / 8)) * 8;
  *reinterpret_cast<u32x4*>(Xf + ws_frag_off(m, k)) = *reinterpret_cast<const u32x4*>(X + (int64_t)m * x_st + k);
}

bool shape_ok(int64_t N, int64_t K, int epi) {
  return N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0 && N / 16 < INT32_MAX && K < INT32_MAX &&
         (epi != kSilu || N % 16 == 0);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_wsgemm_shuffle(const uint16_t* W, int64_t N, int64_t K, int64_t w_row_stride, int pair_halves,
                                    const uint16_t* col_scale, int zero_centred, uint16_t* Wp, void* stream) {
  TRIDA_CHECK(W && Wp, TRIDA_ERR_NULL, "wsgemm_shuffle: W and Wp are required");
  TRIDA_CHECK(N > 0 && K > 0 && N % 16 == 0 && K % 32 == 0 && w_row_stride >= K && w_row_stride % 8 == 0,
              TRIDA_ERR_ARG, "wsgemm_shuffle: need N %% 16 == 0, K %% 32 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  TRIDA_CHECK(((((uintptr_t)W) | (uintptr_t)Wp | (uintptr_t)col_scale) & 15) == 0, TRIDA_ERR_ALIGN,
              "wsgemm_shuffle: 16-byte alignment");
  const int64_t total = N / 16 * (K / 32) * kWave;
  hipLaunchKernelGGL(shuffle_kernel, dim3((unsigned)cdiv(total, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     W, w_row_stride, (int)N, (int)K, pair_halves ? 1 : 0, col_scale, zero_centred ? 1 : 0,
                     reinterpret_cast<u32x4*>(Wp));
  return launch_status("wsgemm_shuffle");
}

extern "C" int trida_wsgemm_plan(int64_t N, int64_t K, int epilogue, int32_t* kgroups) {
  TRIDA_CHECK(kgroups, TRIDA_ERR_NULL, "wsgemm_plan: kgroups is required");
  TRIDA_CHECK(epilogue >= kStore && epilogue <= kSilu, TRIDA_ERR_ARG, "wsgemm_plan: unknown epilogue %d", epilogue);
  TRIDA_CHECK(shape_ok(N, K, epilogue), TRIDA_ERR_ARG, "wsgemm_plan: need N %% 16 == 0, K %% 32 == 0");
  const Plan p = plan_for(N, K, epilogue);
  TRIDA_CHECK(p.cfg >= 0, TRIDA_ERR_ARG, "wsgemm_plan: K too long for one workgroup (epilogue %d needs kg == 1)",
              epilogue);
  *kgroups = p.kg;
  return TRIDA_OK;
}

namespace {
// the weight-streaming GEMM behind every entry point: ss null = no RMSNorm prologue; flags TRIDA_WS_X_FRAG /
// TRIDA_WS_OUT_FRAG select the fragment order of X / of the bf16 output
int ws_run(const char* name, const uint16_t* X, int64_t x_row_stride, const float* ss, float eps, const uint16_t* Wp,
           int64_t M, int64_t N, int64_t K, int epilogue, void* out, int64_t out_row_stride, int flags, void* stream,
           float* pval = nullptr, int* pidx = nullptr, float* psum = nullptr) {
  // argmax (+ confidence) only through trida_wsgemm_argmax (_conf), which pass pval / pidx (/ psum)
  const bool amax = epilogue == kArgmax || epilogue == kArgmaxConf;
  TRIDA_CHECK(X && Wp && (out || amax) && (!amax || (pval && pidx)) && (epilogue != kArgmaxConf || psum),
              TRIDA_ERR_NULL, "%s: X, Wp and out (argmax: pval and pidx; with confidence psum) are required", name);
  TRIDA_CHECK(epilogue >= kStore && epilogue <= (amax ? kArgmaxConf : kSilu), TRIDA_ERR_ARG,
              "%s: unknown epilogue %d", name, epilogue);
  TRIDA_CHECK(!amax || (!ss && !(flags & TRIDA_WS_OUT_FRAG)), TRIDA_ERR_ARG,
              "%s: the argmax epilogue takes no RMSNorm prologue and a row-major output", name);
  TRIDA_CHECK(!ss || epilogue != kParts, TRIDA_ERR_ARG,
              "%s: the RMSNorm prologue takes the bf16 (0) or SwiGLU (2) epilogue", name);
  TRIDA_CHECK((flags & ~(TRIDA_WS_X_FRAG | TRIDA_WS_OUT_FRAG)) == 0 &&
                  (!(flags & TRIDA_WS_OUT_FRAG) || epilogue != kParts),
              TRIDA_ERR_ARG, "%s: bad flags %d (a fragment-order output needs the bf16 or SwiGLU epilogue)", name,
              flags);
  TRIDA_CHECK(M >= 1 && M <= kMaxM && shape_ok(N, K, epilogue), TRIDA_ERR_ARG,
              "%s: need 1 <= M <= %d, N %% 16 == 0, K %% 32 == 0 (M=%lld N=%lld K=%lld)", name, kMaxM, (long long)M,
              (long long)N, (long long)K);
  const bool xf = flags & TRIDA_WS_X_FRAG, of = flags & TRIDA_WS_OUT_FRAG;
  TRIDA_CHECK(!of || (epilogue == kSilu ? N / 2 : N) % 32 == 0, TRIDA_ERR_ARG,
              "%s: a fragment-order output needs a width that is a multiple of 32", name);
  TRIDA_CHECK(xf || (x_row_stride >= K && x_row_stride % 8 == 0), TRIDA_ERR_ARG, "%s: bad X row stride", name);
  TRIDA_CHECK(epilogue == kParts || of || (amax && !out) ||
                  (out_row_stride >= (epilogue == kSilu ? N / 2 : N) && out_row_stride % 4 == 0),
              TRIDA_ERR_ARG, "%s: bad output row stride", name);
  TRIDA_CHECK(!amax || (N <= INT32_MAX && ((uintptr_t)pval & 3) == 0 && ((uintptr_t)pidx & 3) == 0 &&
                        ((uintptr_t)psum & 3) == 0),
              TRIDA_ERR_ARG, "%s: argmax needs N < 2^31 and 4-byte aligned pval / pidx / psum", name);
  TRIDA_CHECK(((((uintptr_t)X) | (uintptr_t)Wp | (uintptr_t)out) & 15) == 0 && ((uintptr_t)ss & 3) == 0,
              TRIDA_ERR_ALIGN, "%s: X, Wp and out must be 16-byte aligned", name);
  const Plan p = plan_for(N, K, epilogue);
  TRIDA_CHECK(p.cfg >= 0 && (!ss || ss_chunks((int)K) <= kMaxSsChunks), TRIDA_ERR_ARG,
              "%s: K too long for one workgroup (epilogue %d needs kg == 1)", name, epilogue);
  WsArgs a{X, reinterpret_cast<const u32x4*>(Wp), out, x_row_stride, out_row_stride, (int)M, (int)N, (int)K, p.T, ss,
           eps, xf ? 1 : 0, of ? 1 : 0, pval, pidx, psum};
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (amax) {
    if (epilogue == kArgmaxConf) launch_cfg<kArgmaxConf, false>(a, p, st);
    else launch_cfg<kArgmax, false>(a, p, st);
  } else if (ss) {
    if (epilogue == kStore) launch_cfg<kStore, true>(a, p, st);
    else launch_cfg<kSilu, true>(a, p, st);
  } else {
    if (epilogue == kStore) launch_cfg<kStore, false>(a, p, st);
    else if (epilogue == kParts) launch_cfg<kParts, false>(a, p, st);
    else launch_cfg<kSilu, false>(a, p, st);
  }
  return launch_status(name);
}
}  // namespace

extern "C" int trida_wsgemm(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M, int64_t N,
                            int64_t K, int epilogue, void* out, int64_t out_row_stride, void* stream) {
  return ws_run("wsgemm", X, x_row_stride, nullptr, 0.f, Wp, M, N, K, epilogue, out, out_row_stride, 0, stream);
}

extern "C" int trida_wsgemm_norm(const uint16_t* X, int64_t x_row_stride, const float* ss, float eps, const uint16_t* Wp,
                                 int64_t M, int64_t N, int64_t K, int epilogue, void* out, int64_t out_row_stride,
                                 void* stream) {
  TRIDA_CHECK(ss, TRIDA_ERR_NULL, "wsgemm_norm: ss is required");
  return ws_run("wsgemm_norm", X, x_row_stride, ss, eps, Wp, M, N, K, epilogue, out, out_row_stride, 0, stream);
}

extern "C" int trida_wsgemm_ex(const uint16_t* X, int64_t x_row_stride, const float* ss, float eps, const uint16_t* Wp,
                               int64_t M, int64_t N, int64_t K, int epilogue, void* out, int64_t out_row_stride,
                               int flags, void* stream) {
  return ws_run("wsgemm_ex", X, x_row_stride, ss, eps, Wp, M, N, K, epilogue, out, out_row_stride, flags, stream);
}

extern "C" int64_t trida_wsgemm_argmax_splits(int64_t N, int64_t K) {
  if (!shape_ok(N, K, kArgmax)) return 0;
  const Plan p = plan_for(N, K, kArgmax);
  return p.cfg < 0 ? 0 : cdiv(N / 16, p.T);
}

extern "C" int trida_wsgemm_argmax(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M, int64_t N,
                                   int64_t K, int flags, uint16_t* logits, int64_t out_row_stride, float* pval,
                                   int32_t* pidx, void* stream) {
  return ws_run("wsgemm_argmax", X, x_row_stride, nullptr, 0.f, Wp, M, N, K, kArgmax, logits, out_row_stride, flags,
                stream, pval, pidx);
}

// the configuration of a per-head-scaled product: every wave's K slice one head of K / heads columns
int headnorm_plan(int64_t N, int64_t K, int64_t heads, Plan* p) {
  TRIDA_CHECK(heads > 0 && K % heads == 0 && (K / heads) % 32 == 0 && shape_ok(N, K, kParts), TRIDA_ERR_ARG,
              "wsgemm_headnorm: need N %% 16 == 0 and heads of a multiple of 32 columns (N=%lld K=%lld heads=%lld)",
              (long long)N, (long long)K, (long long)heads);
  *p = plan_for(N, K, kParts, (int)(K / heads / 32));
  TRIDA_CHECK(p->cfg >= 0, TRIDA_ERR_ARG, "wsgemm_headnorm: no plan takes heads of %lld columns",
              (long long)(K / heads));
  return TRIDA_OK;
}

extern "C" int trida_wsgemm_headnorm_planes(int64_t N, int64_t K, int64_t heads, int32_t* kgroups) {
  TRIDA_CHECK(kgroups, TRIDA_ERR_NULL, "wsgemm_headnorm_planes: kgroups is required");
  Plan p;
  const int rc = headnorm_plan(N, K, heads, &p);
  if (rc != TRIDA_OK) return rc;
  *kgroups = p.kg;
  return TRIDA_OK;
}

extern "C" int trida_wsgemm_headnorm(const uint16_t* Xf, const uint16_t* Wp, int64_t M, int64_t N, int64_t K,
                                     const float* ss_parts, int64_t heads, float eps, float* parts, void* stream) {
  TRIDA_CHECK(Xf && Wp && ss_parts && parts, TRIDA_ERR_NULL, "wsgemm_headnorm: Xf, Wp, ss_parts and parts are required");
  TRIDA_CHECK(M >= 1 && M <= kMaxM, TRIDA_ERR_ARG, "wsgemm_headnorm: need 1 <= M <= %d", kMaxM);
  TRIDA_CHECK(((((uintptr_t)Xf) | (uintptr_t)Wp | (uintptr_t)parts) & 15) == 0 && ((uintptr_t)ss_parts & 3) == 0,
              TRIDA_ERR_ALIGN, "wsgemm_headnorm: Xf, Wp and parts 16-byte aligned, ss_parts 4-byte aligned");
  Plan p;
  const int rc = headnorm_plan(N, K, heads, &p);
  if (rc != TRIDA_OK) return rc;
  WsArgs a{Xf, reinterpret_cast<const u32x4*>(Wp), parts, 0, 0, (int)M, (int)N, (int)K, p.T, nullptr, 0.f, 1, 0,
           nullptr, nullptr, nullptr, ss_parts, (int)heads, eps};
  launch_cfg<kParts, false>(a, p, static_cast<hipStream_t>(stream));
  return launch_status("wsgemm_headnorm");
}

extern "C" int trida_wsgemm_argmax_conf(const uint16_t* X, int64_t x_row_stride, const uint16_t* Wp, int64_t M,
                                        int64_t N, int64_t K, int flags, uint16_t* logits, int64_t out_row_stride,
                                        float* pval, int32_t* pidx, float* psum, void* stream) {
  return ws_run("wsgemm_argmax_conf", X, x_row_stride, nullptr, 0.f, Wp, M, N, K, kArgmaxConf, logits, out_row_stride,
                flags, stream, pval, pidx, psum);
}

extern "C" int64_t trida_ws_frag_elems(int64_t K) { return K > 0 && K % 32 == 0 ? K / 32 * kWsFragMT * 64 * 8 : 0; }

extern "C" int trida_ws_frag(const uint16_t* X, int64_t x_row_stride, int64_t M, int64_t K, uint16_t* Xf, void* stream) {
  TRIDA_CHECK(X && Xf, TRIDA_ERR_NULL, "ws_frag: X and Xf are required");
  TRIDA_CHECK(M >= 1 && M <= kMaxM && K > 0 && K % 32 == 0 && K < INT32_MAX && x_row_stride >= K &&
                  x_row_stride % 8 == 0,
              TRIDA_ERR_ARG, "ws_frag: need 1 <= M <= %d, K %% 32 == 0", kMaxM);
  TRIDA_CHECK(((((uintptr_t)X) | (uintptr_t)Xf) & 15) == 0, TRIDA_ERR_ALIGN, "ws_frag: 16-byte aligned X and Xf");
  hipLaunchKernelGGL(frag_kernel, dim3((unsigned)cdiv(M * (K / 8), 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), X, x_row_stride, (int)M, (int)K, Xf);
  return launch_status("ws_frag");
}

extern "C" int64_t trida_residual_ss_chunks(int64_t dim) { return dim > 0 ? ss_chunks((int)dim) : 0; }

extern "C" int trida_residual_parts(uint16_t* h, int64_t h_row_stride, const float* parts, int64_t n_parts,
                                    int64_t plane_stride, int64_t rows, int64_t dim, float* ss, void* stream) {
  return trida_residual_parts_frag(h, h_row_stride, parts, n_parts, plane_stride, rows, dim, ss, nullptr, stream);
}

extern "C" int trida_residual_parts_frag(uint16_t* h, int64_t h_row_stride, const float* parts, int64_t n_parts,
                                         int64_t plane_stride, int64_t rows, int64_t dim, float* ss, uint16_t* h_frag,
                                         void* stream) {
  TRIDA_CHECK(h && ss && (parts || n_parts == 0), TRIDA_ERR_NULL, "residual_parts: h and ss (and parts) are required");
  TRIDA_CHECK(!h_frag || (rows <= kMaxM && dim % 32 == 0 && ((uintptr_t)h_frag & 15) == 0), TRIDA_ERR_ARG,
              "residual_parts: a fragment-order copy needs rows <= %d, dim %% 32 == 0 and 16-byte alignment", kMaxM);
  TRIDA_CHECK(rows > 0 && rows < INT32_MAX && dim > 0 && dim % 4 == 0 && dim < INT32_MAX && n_parts >= 0 &&
                  n_parts <= 64 && (n_parts == 0 || plane_stride >= rows * dim) && h_row_stride >= dim,
              TRIDA_ERR_ARG, "residual_parts: bad sizes (dim %% 4 == 0, 0 <= n_parts <= 64)");
  TRIDA_CHECK(((uintptr_t)h & 7) == 0 && h_row_stride % 4 == 0 && ((uintptr_t)parts & 15) == 0 && plane_stride % 4 == 0,
              TRIDA_ERR_ALIGN, "residual_parts: h rows 8-byte and parts 16-byte aligned");
  hipLaunchKernelGGL(residual_kernel, dim3((unsigned)rows, (unsigned)ss_chunks((int)dim)), dim3(kWave), 0,
                     static_cast<hipStream_t>(stream), h, h_row_stride, parts, (int)n_parts, plane_stride, (int)dim, ss,
                     h_frag);
  return launch_status("residual_parts");
}
