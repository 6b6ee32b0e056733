// Greedy self-spec acceptance: one HBM pass over the verify logits, then a per-sequence prefix scan.
//
// Two launches on the caller's stream, no atomics:
//   split_argmax (grid S x R x B): block (s, r, b) reduces split s of row r of sequence b to an
//       (argmax value, index) pair in scratch. Each thread issues U 16-byte loads per tile
//       back to back (indices clamped in bounds, loads past the split set to -inf), so a block has
//       U * 4 KiB in flight, and folds the tile as a max first and an index search only when the
//       tile's max beats the thread's best.
//   finalize (grid B): stages the split results and the drafts through LDS (one memory latency per
//       pass), reduces each row with one thread per row, then one wave ballots draft matches and
//       takes the accepted length as the count of leading ones.
// A single-launch variant that elected the last block with device-scope counters measured slower on
// gfx950: every arrive costs a device-scope atomic round trip (~20 ns each, serialised), which for
// ~600 blocks exceeds the whole streaming pass.
#include <limits.h>
#include <math.h>

#include <mutex>

#include "common.h"

namespace trida {

// Scratch of the allocation-free entry point (trida_greedy_accept_noalloc): the split results of the
// streaming pass, in a file-scope device array. Every GPU the library runs on holds its own copy at its
// own address until the process ends; host code reaches it only through the address that
// hipGetSymbolAddress returns for that GPU (the array's name is a host-side stand-in). The split
// results are written before they are read, so nothing in it needs clearing between calls.
namespace noalloc {
constexpr int64_t kScratchBytes = TRIDA_GREEDY_ACCEPT_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
}  // namespace noalloc

namespace {

constexpr int kThreads = 256;
constexpr int kStage = 2048;  // split results staged per pass by finalize (a pass holds whole rows)

// (a, ia) ranks above (b, ib): NaN above everything, then larger value, then smaller index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) { return argmax_better(a, ia, b, ib); }

__device__ __forceinline__ void wave_argbest(float& v, int& i) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(v, off, kWave);
    const int oi = __shfl_xor(i, off, kWave);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Within one thread indices only increase, so a strict "greater (or first NaN)" test keeps the first
// occurrence. Branch-free (selects only), so a tile's loads stay in flight together.
__device__ __forceinline__ void take(float x, int ix, bool valid, float& v, int& i) {
  const bool t = valid && (v == v) && ((x != x) || (x > v));
  v = t ? x : v;
  i = t ? ix : i;
}

struct SplitArgs {
  const void* logits;
  int64_t batch_stride, row_stride;  // elements
  int V, R, S, chunk;
  float* pval;
  int* pidx;
  float* psum;  // sum of exp(x - split max), or null
};

template <typename TIn>
struct Vec;  // one 16-byte load
template <>
struct Vec<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void get(const u32x4 w, float* f) {
    f[0] = __uint_as_float(w.x);
    f[1] = __uint_as_float(w.y);
    f[2] = __uint_as_float(w.z);
    f[3] = __uint_as_float(w.w);
  }
  __device__ __forceinline__ static float one(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
};
template <>
struct Vec<uint16_t> {  // bf16
  static constexpr int N = 8;
  __device__ __forceinline__ static void get(const u32x4 w, float* f) {
    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f[2 * j] = __uint_as_float(ws[j] << 16);
      f[2 * j + 1] = __uint_as_float(ws[j] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static float one(const void* p, int64_t i) {
    return bf2f(static_cast<const uint16_t*>(p)[i]);
  }
};

// Element e of load u of a tile, as fp32.
template <typename TIn>
__device__ __forceinline__ float elem(const u32x4 w, int e) {
  const uint32_t word = w[Vec<TIn>::N == 4 ? e : e >> 1];
  if (Vec<TIn>::N == 4) return __uint_as_float(word);
  return __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
}

// Folds one tile (U loads of N elements per thread; row4 + j0 + u * kThreads is load u) into the
// thread's running (best, bi), with take()'s result: per load the max m_u, then the tile max m; only
// when m beats best does the thread find the first load holding m and the first element of it equal
// to m (+-inf need nothing more: -inf never beats best, and the first +inf is the first element equal
// to m). A NaN is flagged from the raw words (|x| above inf, i.e. x << 1 above inf << 1 per element)
// and such a tile (rare) is read again and taken element by element. Loads at or past n4 hold -inf;
// element e of load u has index ix0 + u * N * kThreads + e.
// kConf: the tile's softmax partial sum(exp(x - m)) is folded into the thread's (sm, ss) once per tile;
// a tile whose max is +inf is also taken element by element (acc_exp's order for infinities).
template <int U, typename TIn, bool kConf>
__device__ __forceinline__ void fold_tile(const u32x4 (&x)[U], const u32x4* row4, int j0, int n4, int ix0,
                                          float& best, int& bi, float& sm, float& ss) {
  constexpr int N = Vec<TIn>::N;
  constexpr float kLog2e = 1.44269504f;
  float mu[U];
  uint32_t nb = 0u;
  float pm = -INFINITY, ps[4] = {0.f, 0.f, 0.f, 0.f};  // kConf: the tile's running (max, sum exp(x - max))
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float m = elem<TIn>(x[u], 0);
#pragma unroll
    for (int e = 1; e < N; ++e) m = fmaxf(m, elem<TIn>(x[u], e));
    mu[u] = m;
#pragma unroll
    for (int k = 0; k < 4; ++k)  // bf16: both halves' magnitudes at the top of a word
      nb = N == 8 ? max(nb, max(x[u][k] << 1, x[u][k] << 17)) : max(nb, x[u][k] << 1);
    if (kConf) {  // rescale to the new max, then add this load's terms while its elements are live
      const float nm = fmaxf(pm, m);
      const float sc = pm > -INFINITY ? __builtin_amdgcn_exp2f((pm - nm) * kLog2e) : 0.f;
      const float ml = nm > -INFINITY ? nm * kLog2e : 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) ps[k] *= sc;
#pragma unroll
      for (int e = 0; e < N; ++e) ps[e & 3] += __builtin_amdgcn_exp2f(fmaf(elem<TIn>(x[u], e), kLog2e, -ml));
      pm = nm;
    }
  }
  float m = mu[0];
#pragma unroll
  for (int u = 1; u < U; ++u) m = fmaxf(m, mu[u]);
  if (nb > (N == 8 ? 0xff01ffffu : 0xff000000u) || (kConf && m == INFINITY)) {  // a NaN (or +inf) in the tile
#pragma unroll 1
    for (int u = 0; u < U; ++u) {
      const int j = j0 + u * kThreads;
      if (j >= n4) break;
      const u32x4 w = row4[j];
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const float f = elem<TIn>(w, e);
        take(f, ix0 + u * N * kThreads + e, true, best, bi);
        if (kConf) acc_exp(f, true, sm, ss);
      }
    }
    return;
  }
  if (kConf && m > -INFINITY) {  // pm == m
    const float st = (ps[0] + ps[1]) + (ps[2] + ps[3]);
    if (m > sm) {
      ss = ss * __expf(sm - m) + st;
      sm = m;
    } else {
      ss += st * __expf(m - sm);
    }
  }
  if (!(m > best)) return;  // also keeps a NaN best
  const int ustride = N * kThreads;
  int us = U - 1;
#pragma unroll
  for (int u = U - 2; u >= 0; --u) us = mu[u] == m ? u : us;
  u32x4 w = x[U - 1];
#pragma unroll
  for (int u = U - 2; u >= 0; --u) w = u == us ? x[u] : w;
  int es = N - 1;
#pragma unroll
  for (int e = N - 2; e >= 0; --e) es = elem<TIn>(w, e) == m ? e : es;
  best = m;
  bi = ix0 + us * ustride + es;
}

template <int U, bool kVec, typename TIn, bool kConf>
__global__ __launch_bounds__(kThreads) void split_argmax_kernel(SplitArgs a) {
  constexpr int N = Vec<TIn>::N;
  const int s = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int64_t row_off = (int64_t)b * a.batch_stride + (int64_t)r * a.row_stride;
  const TIn* row = static_cast<const TIn*>(a.logits) + row_off;
  const int lo = s * a.chunk;
  const int hi = min(a.V, lo + a.chunk);

  float best = -INFINITY, sm = -INFINITY, ss = 0.f;
  int bi = INT_MAX;
  if (kVec) {
    // lo is a multiple of N and the row start is 16-byte aligned (checked on the host)
    const u32x4* row4 = reinterpret_cast<const u32x4*>(row + lo);
    const int n4 = (hi - lo) / N;
    for (int base = 0; base < n4; base += kThreads * U) {
      u32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = row4[min(base + u * kThreads + tid, n4 - 1)];
      if (base + U * kThreads > n4) {  // the split's last tile: loads past it become -inf
        const uint32_t ninf = N == 4 ? 0xff800000u : 0xff80ff80u;
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (base + u * kThreads + tid >= n4) x[u] = u32x4{ninf, ninf, ninf, ninf};
      }
      fold_tile<U, TIn, kConf>(x, row4, base + tid, n4, lo + N * (base + tid), best, bi, sm, ss);
    }
    for (int ix = lo + N * n4 + tid; ix < hi; ix += kThreads) {
      const float f = Vec<TIn>::one(row, ix);
      take(f, ix, true, best, bi);
      if (kConf) acc_exp(f, true, sm, ss);
    }
  } else {
    for (int ix = lo + tid; ix < hi; ix += kThreads) {
      const float f = Vec<TIn>::one(row, ix);
      take(f, ix, true, best, bi);
      if (kConf) acc_exp(f, true, sm, ss);
    }
  }

  __shared__ float sv[kThreads / kWave], sx[kThreads / kWave], sy[kThreads / kWave];
  __shared__ int si[kThreads / kWave];
  wave_argbest(best, bi);
  if (kConf) {
    // merge (m, s) pairs across the wave
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float om = __shfl_xor(sm, off, kWave), os = __shfl_xor(ss, off, kWave);
      const float nm = fmaxf(sm, om);
      ss = (nm == -INFINITY) ? 0.f : ss * __expf(sm - nm) + os * __expf(om - nm);
      sm = nm;
    }
  }
  const int wave = tid / kWave, lane = tid % kWave;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
    sx[wave] = sm;
    sy[wave] = ss;
  }
  __syncthreads();
  if (tid == 0) {
    float v = sv[0];
    int i = si[0];
    for (int w = 1; w < kThreads / kWave; ++w)
      if (better(sv[w], si[w], v, i)) {
        v = sv[w];
        i = si[w];
      }
    const int64_t slot = ((int64_t)b * a.R + r) * a.S + s;
    a.pval[slot] = v;
    a.pidx[slot] = i;
    if (kConf) {
      float m = sx[0], sum = sy[0];
      for (int w = 1; w < kThreads / kWave; ++w) {
        const float nm = fmaxf(m, sx[w]);
        sum = (nm == -INFINITY) ? 0.f : sum * __expf(m - nm) + sy[w] * __expf(sx[w] - nm);
        m = nm;
      }
      // stored relative to the split's argmax value (the row max is found among these)
      a.psum[slot] = (m == -INFINITY || v != v) ? 0.f : sum * __expf(m - v);
    }
  }
}

struct FinalArgs {
  const float* pval;
  const int* pidx;
  int R, S;
  const int64_t* drafts;
  int64_t draft_stride;
  int K;
  const int32_t* n_live;
  const int64_t* ctx_len;
  int64_t* argmax_out;
  int32_t* n_acc;
  int64_t* bonus;
  int64_t* crop;
};

__device__ void accept_scan(const FinalArgs& a, int b, const int* s_am, const long long* s_dr, int lane);

__global__ __launch_bounds__(kThreads) void finalize_kernel(FinalArgs a) {
  const int b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  __shared__ float s_pv[kStage];
  __shared__ int s_pi[kStage];
  __shared__ int s_am[1024];
  __shared__ long long s_dr[1024];
  const int64_t pbase = (int64_t)b * a.R * a.S;
  for (int k0 = tid; k0 < a.K; k0 += kThreads) s_dr[k0] = a.drafts[(int64_t)b * a.draft_stride + k0];
  const int rows_per_pass = kStage / a.S;  // the host keeps S <= kStage
  for (int r0 = 0; r0 < a.R; r0 += rows_per_pass) {
    const int nr = min(rows_per_pass, a.R - r0);
    const int c0 = r0 * a.S, cn = nr * a.S;
    float pv[kStage / kThreads];
    int pi[kStage / kThreads];
#pragma unroll
    for (int u = 0; u < kStage / kThreads; ++u) {
      const int j = min(u * kThreads + tid, cn - 1);
      pv[u] = a.pval[pbase + c0 + j];
      pi[u] = a.pidx[pbase + c0 + j];
    }
#pragma unroll
    for (int u = 0; u < kStage / kThreads; ++u) {
      const int j = u * kThreads + tid;
      if (j < cn) {
        s_pv[j] = pv[u];
        s_pi[j] = pi[u];
      }
    }
    __syncthreads();
    // one thread per row scans its splits in LDS (no cross-lane shuffles on the critical path)
    for (int rr = r0 + tid; rr < r0 + nr; rr += kThreads) {
      const int j0 = (rr - r0) * a.S;
      float v = s_pv[j0];
      int i = s_pi[j0];
      for (int ss = 1; ss < a.S; ++ss)
        if (better(s_pv[j0 + ss], s_pi[j0 + ss], v, i)) {
          v = s_pv[j0 + ss];
          i = s_pi[j0 + ss];
        }
      if (i == INT_MAX) i = 0;  // a row that is all -inf keeps index 0, as torch.argmax does
      s_am[rr] = i;
      if (a.argmax_out) a.argmax_out[(int64_t)b * a.R + rr] = i;
    }
    __syncthreads();
  }

  if (wave == 0) accept_scan(a, b, s_am, s_dr, lane);
}

// Many splits per row (the LM head's argmax epilogue leaves one per workgroup, ~255): 16 waves, each taking
// rows wave, wave + 16, ... two at a time, its lanes striding over a row's splits with coalesced loads; every
// load of the two rows' first 256 splits is issued before any is compared (one memory latency per pair of
// rows instead of one per split step), then a wave reduction; the same scan.
constexpr int kWideThreads = 1024;
__global__ __launch_bounds__(kWideThreads) void wide_finalize_kernel(FinalArgs a) {
  constexpr int NWV = kWideThreads / kWave, PER = 4;  // waves; splits per lane per pass
  const int b = blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  __shared__ int s_am[1024];
  __shared__ long long s_dr[1024];
  for (int k0 = tid; k0 < a.K; k0 += kWideThreads) s_dr[k0] = a.drafts[(int64_t)b * a.draft_stride + k0];
  const int64_t total = (int64_t)a.R * a.S;  // pairs of this sequence
  for (int r0 = wave; r0 < a.R; r0 += 2 * NWV) {
    float v[2] = {-INFINITY, -INFINITY};
    int i[2] = {INT_MAX, INT_MAX};
    for (int s0 = 0; s0 < a.S; s0 += PER * kWave) {
      float pv[2][PER];
      int pi[2][PER];
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < PER; ++j) {  // clamped, unconditional loads; out-of-range pairs are masked below
          const int64_t e = min((int64_t)(r0 + u * NWV) * a.S + s0 + j * kWave + lane, total - 1);
          pv[u][j] = a.pval[(int64_t)b * total + e];
          pi[u][j] = a.pidx[(int64_t)b * total + e];
        }
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int j = 0; j < PER; ++j)  // a lane's splits come in column order
          if (s0 + j * kWave + lane < a.S && better(pv[u][j], pi[u][j], v[u], i[u])) {
            v[u] = pv[u][j];
            i[u] = pi[u][j];
          }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = r0 + u * NWV;
      wave_argbest(v[u], i[u]);
      if (lane == 0 && r < a.R) {
        const int x = i[u] == INT_MAX ? 0 : i[u];  // a row that is all -inf keeps index 0, as torch.argmax does
        s_am[r] = x;
        if (a.argmax_out) a.argmax_out[(int64_t)b * a.R + r] = x;
      }
    }
  }
  __syncthreads();
  if (wave == 0) accept_scan(a, b, s_am, s_dr, lane);
}

// A denoise pass's readout from the per-split (max, index, sum exp(x - max)) triples of the LM head's argmax +
// confidence epilogue: per row, the argmax over the splits and the softmax probability of the argmax,
// 1 / sum_s psum_s e^{pval_s - max}. Block = one sequence (16 waves, a wave per row; two rows per wave per
// pass, every split load of both rows issued before the compares). S <= 256: one pass, the sum from the
// same loads.
constexpr int kConfPer = 4;
__global__ __launch_bounds__(kWideThreads) void conf_finalize_kernel(const float* pval, const int* pidx,
                                                                     const float* psum, int R, int S, int64_t* argmax,
                                                                     float* conf, int64_t out_st) {
  constexpr int NWV = kWideThreads / kWave;
  const int b = blockIdx.x, wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int64_t total = (int64_t)R * S, base = (int64_t)b * total;
  for (int r0 = wave; r0 < R; r0 += 2 * NWV) {
    float pv[2][kConfPer], ps[2][kConfPer];
    int pi[2][kConfPer];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < kConfPer; ++j) {  // clamped, unconditional loads; out-of-range splits are masked below
        const int64_t e = min((int64_t)(r0 + u * NWV) * S + j * kWave + lane, total - 1);
        pv[u][j] = pval[base + e];
        pi[u][j] = pidx[base + e];
        ps[u][j] = psum[base + e];
      }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int r = r0 + u * NWV;
      float v = -INFINITY;
      int i = INT_MAX;
#pragma unroll
      for (int j = 0; j < kConfPer; ++j)  // a lane's splits come in column order
        if (j * kWave + lane < S && better(pv[u][j], pi[u][j], v, i)) {
          v = pv[u][j];
          i = pi[u][j];
        }
      wave_argbest(v, i);  // every lane holds the row's (max, index)
      float sum = 0.f;
#pragma unroll
      for (int j = 0; j < kConfPer; ++j)
        if (j * kWave + lane < S) sum += ps[u][j] * __expf(pv[u][j] - v);
      sum = wave_sum(sum);
      if (lane == 0 && r < R) {
        argmax[(int64_t)b * out_st + r] = i == INT_MAX ? 0 : i;  // an all -inf row keeps index 0
        conf[(int64_t)b * out_st + r] = sum > 0.f ? 1.f / sum : 0.f;
      }
    }
  }
}

// wave 0 of a finalize block: prefix scan of draft matches (ballot; accepted = count of leading ones)
__device__ void accept_scan(const FinalArgs& a, int b, const int* s_am, const long long* s_dr, int lane) {
  {
    const int live = a.n_live ? min(max(a.n_live[b], 0), a.K) : a.K;
    int n_acc = 0;
    bool open = true;
    for (int j0 = 0; j0 < a.K && open; j0 += kWave) {
      const int j = j0 + lane;
      bool match = false;
      if (j < a.K) match = (j < live) && ((long long)s_am[j] == s_dr[j]);
      const unsigned long long lead = ~__ballot(match);  // first zero bit = first rejected draft
      if (lead == 0ull) {
        n_acc += kWave;
      } else {
        n_acc += __builtin_ctzll(lead);
        open = false;
      }
    }
    n_acc = min(n_acc, a.K);
    if (lane == 0) {
      a.n_acc[b] = n_acc;
      a.bonus[b] = s_am[n_acc];
      const int64_t ctx = a.ctx_len ? a.ctx_len[b] : 0;
      a.crop[b] = ctx + 1 + n_acc;
    }
  }
}

// one thread per row: argmax over the splits and the softmax probability of the argmax
__global__ __launch_bounds__(256) void row_finalize_kernel(const float* pval, const int* pidx, const float* psum,
                                                           int rows, int S, int64_t* argmax, float* conf) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int64_t base = (int64_t)r * S;
  float v = pval[base];
  int i = pidx[base];
  for (int s = 1; s < S; ++s)
    if (better(pval[base + s], pidx[base + s], v, i)) {
      v = pval[base + s];
      i = pidx[base + s];
    }
  if (i == INT_MAX) i = 0;
  argmax[r] = i;
  if (conf) {
    float sum = 0.f;
    for (int s = 0; s < S; ++s) sum += psum[base + s] * __expf(pval[base + s] - v);
    conf[r] = sum > 0.f ? 1.f / sum : 0.f;
  }
}

// The unmasking of a denoise pass: per sequence, the `count` MASK slots with the highest confidence
// (ties: the lower slot first, as a stable descending sort) take their shifted prediction (row j
// predicts slot j + 1) and leave the mask. One block per sequence; a slot's rank is the number of
// slots ahead of it in that order, so the chosen slots are those ranked below count.
constexpr int kMaxUnmask = 1024;
__global__ __launch_bounds__(256) void unmask_top_kernel(const int64_t* am, const float* conf, int64_t ac_st,
                                                         uint8_t* masked, int64_t* canvas, int64_t cv_st, int blk,
                                                         int count) {
  __shared__ float s_sc[kMaxUnmask];
  const int64_t b = blockIdx.x;
  for (int j = threadIdx.x; j < blk; j += blockDim.x) s_sc[j] = masked[b * blk + j] ? conf[b * ac_st + j] : -INFINITY;
  __syncthreads();
  for (int j = threadIdx.x; j < blk; j += blockDim.x) {
    const float sj = s_sc[j];
    int rank = 0;
    for (int i = 0; i < blk; ++i) rank += (s_sc[i] > sj) | ((s_sc[i] == sj) & (i < j));
    if (rank < count) {
      canvas[b * cv_st + j + 1] = am[b * ac_st + j];
      masked[b * blk + j] = 0;
    }
  }
}

// One sequence per thread: the host decision of a bd_bidir_shift self-spec step, taken on the device so
// that a whole step (canvas forward, acceptance, this, the rollback) replays from one graph.
__global__ __launch_bounds__(64) void canvas_advance_kernel(const int64_t* am, int64_t am_st, const int32_t* n_acc,
                                                            int64_t* canvas, int64_t cv_st, uint8_t* verify,
                                                            int32_t* n_keep, int64_t* emit, int32_t* n_emit,
                                                            int64_t* committed, int32_t* kind, int B, int N,
                                                            int64_t mask_id) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  const int64_t* a = am + (int64_t)b * am_st;
  int64_t* cv = canvas + (int64_t)b * cv_st;
  int64_t* em = emit + (int64_t)b * N;
  int64_t* cm = committed + (int64_t)b * N;
  const int blk = 2 * N - 1;
  const bool ver = verify[b] != 0;
  kind[b] = ver ? 1 : 0;
  if (!ver) {  // cold start [t0, MASK...]: emit the clean token, its row's successors become the specs
    em[0] = a[0];
    n_emit[b] = 1;
    cm[0] = cv[0];
    n_keep[b] = 1;
    cv[0] = a[0];
    for (int j = 1; j < N; ++j) cv[j] = a[j];
    for (int j = N; j < blk; ++j) cv[j] = mask_id;
    verify[b] = 1;
    return;
  }
  const int acc = min(max(n_acc[b], 0), N - 1);
  cm[0] = cv[0];
  for (int j = 0; j < acc; ++j) {
    em[j] = cv[1 + j];
    cm[1 + j] = cv[1 + j];
  }
  n_keep[b] = 1 + acc;
  if (acc < N - 1) {  // rejected at spec acc: the correction, then a cold start from it
    em[acc] = a[acc];
    n_emit[b] = acc + 1;
    cv[0] = a[acc];
    for (int j = 1; j < blk; ++j) cv[j] = mask_id;
    verify[b] = 0;
  } else {  // every spec accepted: the clean token, and the MASK rows' predictions as the next specs
    em[N - 1] = a[N - 1];
    n_emit[b] = N;
    cv[0] = a[N - 1];
    for (int j = 1; j < N; ++j) cv[j] = a[N - 1 + j];
    for (int j = N; j < blk; ++j) cv[j] = mask_id;
    verify[b] = 1;
  }
}

// Split a row into chunks of one tile each (kThreads * U float4), U in {4, 8, 16}: the largest U
// that still gives at least ~512 blocks; callers may force the split count.
void plan(int64_t B, int64_t R, int64_t V, int64_t splits_req, int elems, int64_t* S, int64_t* chunk) {
  int64_t c;
  if (splits_req > 0) {
    c = align_up(cdiv(V, splits_req), 8);
  } else {
    c = (int64_t)elems * kThreads * 4;
    for (int u = 16; u >= 4; u /= 2) {
      c = (int64_t)elems * kThreads * u;
      if (B * R * cdiv(V, c) >= 512) break;
    }
  }
  *chunk = c;
  *S = cdiv(V, c);
}

int pick_unroll(int64_t chunk, int elems) {
  const int64_t per_thread = cdiv(chunk / elems, kThreads);
  return per_thread <= 4 ? 4 : (per_thread <= 8 ? 8 : 16);
}

int64_t scratch_bytes(int64_t B, int64_t R, int64_t S) { return align_up(B * R * S * 4, 256) * 3; }

int elems_of(int dtype) { return dtype == 1 ? 8 : 4; }

template <typename TIn, bool kConf>
int launch_split(const SplitArgs& sa, dim3 grid, bool vec, int64_t chunk, hipStream_t st) {
  if (!vec) {
    hipLaunchKernelGGL((split_argmax_kernel<4, false, TIn, kConf>), grid, dim3(kThreads), 0, st, sa);
  } else {
    switch (pick_unroll(chunk, Vec<TIn>::N)) {
      case 4: hipLaunchKernelGGL((split_argmax_kernel<4, true, TIn, kConf>), grid, dim3(kThreads), 0, st, sa); break;
      case 8: hipLaunchKernelGGL((split_argmax_kernel<8, true, TIn, kConf>), grid, dim3(kThreads), 0, st, sa); break;
      default: hipLaunchKernelGGL((split_argmax_kernel<16, true, TIn, kConf>), grid, dim3(kThreads), 0, st, sa); break;
    }
  }
  return launch_status("split_argmax");
}

// shared planning + first launch of greedy_accept and row_argmax
int run_split(const void* logits, int dtype, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
              int64_t row_stride, bool conf, void* scratch, int64_t scratch_bytes_, int64_t splits, hipStream_t st,
              int64_t* S_out, float** pval, int** pidx, float** psum) {
  TRIDA_CHECK(dtype == 0 || dtype == 1, TRIDA_ERR_ARG, "logits dtype must be 0 (fp32) or 1 (bf16)");
  int64_t S, chunk;
  plan(B, R, V, splits, elems_of(dtype), &S, &chunk);
  TRIDA_CHECK(S <= kStage && S <= 65535, TRIDA_ERR_ARG, "at most %d splits per row", kStage);
  TRIDA_CHECK(scratch_bytes_ >= scratch_bytes(B, R, S), TRIDA_ERR_WORKSPACE, "scratch %lld < %lld bytes",
              (long long)scratch_bytes_, (long long)scratch_bytes(B, R, S));
  char* ws = static_cast<char*>(scratch);
  const int64_t part = align_up(B * R * S * 4, 256);
  *pval = reinterpret_cast<float*>(ws);
  *pidx = reinterpret_cast<int*>(ws + part);
  *psum = reinterpret_cast<float*>(ws + 2 * part);
  *S_out = S;
  SplitArgs sa{logits, batch_stride, row_stride, (int)V, (int)R, (int)S, (int)chunk, *pval, *pidx,
               conf ? *psum : nullptr};
  const int align = elems_of(dtype);
  const bool vec = ((reinterpret_cast<uintptr_t>(logits) & 15) == 0) && (row_stride % align == 0) &&
                   (batch_stride % align == 0) && (chunk % align == 0);
  const dim3 grid((unsigned)S, (unsigned)R, (unsigned)B);
  if (dtype == 0)
    return conf ? launch_split<float, true>(sa, grid, vec, chunk, st) : launch_split<float, false>(sa, grid, vec, chunk, st);
  return conf ? launch_split<uint16_t, true>(sa, grid, vec, chunk, st) : launch_split<uint16_t, false>(sa, grid, vec, chunk, st);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_greedy_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int dtype, int64_t splits) {
  if (B <= 0 || R <= 0 || V <= 0) return 0;
  int64_t S, chunk;
  plan(B, R, V, splits, elems_of(dtype), &S, &chunk);
  return scratch_bytes(B, R, S);
}

extern "C" int trida_greedy_accept(const void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                                   int64_t batch_stride, int64_t row_stride, const int64_t* drafts,
                                   int64_t K, int64_t draft_stride, const int32_t* n_live,
                                   const int64_t* ctx_len, int64_t* argmax_out, int32_t* n_acc,
                                   int64_t* bonus, int64_t* crop, void* scratch, int64_t scratch_bytes_,
                                   int64_t splits, void* stream) {
  TRIDA_CHECK(logits && n_acc && bonus && crop && scratch, TRIDA_ERR_NULL,
              "greedy_accept: logits, n_acc, bonus, crop and scratch are required");
  TRIDA_CHECK(B > 0 && R > 0 && V > 0 && V < INT_MAX && K >= 0, TRIDA_ERR_ARG,
              "greedy_accept: bad sizes B=%lld R=%lld V=%lld K=%lld", (long long)B, (long long)R,
              (long long)V, (long long)K);
  TRIDA_CHECK(R >= K + 1, TRIDA_ERR_ARG, "greedy_accept: need R >= K + 1 (R=%lld K=%lld)", (long long)R,
              (long long)K);
  TRIDA_CHECK(R <= 1024 && B <= 65535, TRIDA_ERR_ARG, "greedy_accept: R <= 1024 and B <= 65535 supported");
  TRIDA_CHECK(K == 0 || drafts, TRIDA_ERR_NULL, "greedy_accept: drafts is NULL with K > 0");
  TRIDA_CHECK(row_stride >= V && batch_stride >= 0, TRIDA_ERR_ARG, "greedy_accept: bad strides");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t S;
  float *pval, *psum;
  int* pidx;
  int rc = run_split(logits, dtype, B, R, V, batch_stride, row_stride, false, scratch, scratch_bytes_, splits, st,
                     &S, &pval, &pidx, &psum);
  if (rc) return rc;
  FinalArgs fa{pval, pidx, (int)R, (int)S, drafts, draft_stride, (int)K, n_live, ctx_len,
               argmax_out, n_acc, bonus, crop};
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)B), dim3(kThreads), 0, st, fa);
  return launch_status("greedy_accept/finalize");
}

extern "C" int trida_greedy_accept_splits(const float* pval, const int32_t* pidx, int64_t B, int64_t R, int64_t S,
                                          const int64_t* drafts, int64_t K, int64_t draft_stride,
                                          const int32_t* n_live, const int64_t* ctx_len, int64_t* argmax_out,
                                          int32_t* n_acc, int64_t* bonus, int64_t* crop, void* stream) {
  TRIDA_CHECK(pval && pidx && n_acc && bonus && crop, TRIDA_ERR_NULL,
              "greedy_accept_splits: pval, pidx, n_acc, bonus and crop are required");
  TRIDA_CHECK(B > 0 && R > 0 && K >= 0 && S >= 1 && S <= kStage, TRIDA_ERR_ARG,
              "greedy_accept_splits: bad sizes B=%lld R=%lld S=%lld (1 <= S <= %d) K=%lld", (long long)B, (long long)R,
              (long long)S, kStage, (long long)K);
  TRIDA_CHECK(R >= K + 1, TRIDA_ERR_ARG, "greedy_accept_splits: need R >= K + 1 (R=%lld K=%lld)", (long long)R,
              (long long)K);
  TRIDA_CHECK(R <= 1024 && B <= 65535, TRIDA_ERR_ARG, "greedy_accept_splits: R <= 1024 and B <= 65535 supported");
  TRIDA_CHECK(K == 0 || drafts, TRIDA_ERR_NULL, "greedy_accept_splits: drafts is NULL with K > 0");
  FinalArgs fa{pval, reinterpret_cast<const int*>(pidx), (int)R, (int)S, drafts, draft_stride, (int)K, n_live, ctx_len,
               argmax_out, n_acc, bonus, crop};
  hipLaunchKernelGGL(wide_finalize_kernel, dim3((unsigned)B), dim3(kWideThreads), 0, static_cast<hipStream_t>(stream), fa);
  return launch_status("greedy_accept_splits");
}

extern "C" int trida_argmax_conf_splits(const float* pval, const int32_t* pidx, const float* psum, int64_t B,
                                        int64_t R, int64_t S, int64_t* argmax, float* conf, int64_t out_row_stride,
                                        void* stream) {
  TRIDA_CHECK(pval && pidx && psum && argmax && conf, TRIDA_ERR_NULL,
              "argmax_conf_splits: pval, pidx, psum, argmax and conf are required");
  TRIDA_CHECK(B > 0 && B <= 65535 && R > 0 && S >= 1 && S <= kConfPer * kWave && out_row_stride >= R,
              TRIDA_ERR_ARG, "argmax_conf_splits: bad sizes B=%lld R=%lld S=%lld (1 <= S <= %d) row stride %lld",
              (long long)B, (long long)R, (long long)S, kConfPer * kWave, (long long)out_row_stride);
  hipLaunchKernelGGL(conf_finalize_kernel, dim3((unsigned)B), dim3(kWideThreads), 0, static_cast<hipStream_t>(stream),
                     pval, reinterpret_cast<const int*>(pidx), psum, (int)R, (int)S, argmax, conf, out_row_stride);
  return launch_status("argmax_conf_splits");
}

namespace {
// Device address of noalloc::scratch per GPU, looked up once per device (with that device current)
// on the first call that runs there.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int noalloc_scratch(hipStream_t st, void** out) {
  int dev = -1;
  hipError_t e = hipStreamGetDevice(st, &dev);
  TRIDA_CHECK(e == hipSuccess, TRIDA_ERR_LAUNCH, "greedy_accept_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
  TRIDA_CHECK(dev >= 0 && dev < kMaxDevices, TRIDA_ERR_ARG, "greedy_accept_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    e = hipGetDevice(&cur);
    TRIDA_CHECK(e == hipSuccess, TRIDA_ERR_LAUNCH, "greedy_accept_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (cur != dev) {
      e = hipSetDevice(dev);
      TRIDA_CHECK(e == hipSuccess, TRIDA_ERR_LAUNCH, "greedy_accept_noalloc: hipSetDevice: %s", hipGetErrorString(e));
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc::scratch));
    if (cur != dev) {
      const hipError_t e2 = hipSetDevice(cur);
      TRIDA_CHECK(e2 == hipSuccess, TRIDA_ERR_LAUNCH, "greedy_accept_noalloc: hipSetDevice: %s",
                  hipGetErrorString(e2));
    }
    TRIDA_CHECK(e == hipSuccess && p, TRIDA_ERR_LAUNCH, "greedy_accept_noalloc: hipGetSymbolAddress: %s",
                hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return TRIDA_OK;
}
}  // namespace

extern "C" int trida_greedy_accept_noalloc(const void* logits, int dtype, int64_t B, int64_t R, int64_t V,
                                           int64_t batch_stride, int64_t row_stride, const int64_t* drafts,
                                           int64_t K, int64_t draft_stride, const int32_t* n_live,
                                           const int64_t* ctx_len, int64_t* argmax_out, int32_t* n_acc,
                                           int64_t* bonus, int64_t* crop, int64_t splits, void* stream) {
  TRIDA_CHECK(dtype == 0 || dtype == 1, TRIDA_ERR_ARG, "greedy_accept_noalloc: logits dtype must be 0 (fp32) or 1 (bf16)");
  TRIDA_CHECK(B > 0 && R > 0 && V > 0 && V < INT_MAX, TRIDA_ERR_ARG, "greedy_accept_noalloc: bad sizes B=%lld R=%lld V=%lld",
              (long long)B, (long long)R, (long long)V);
  const int64_t need = trida_greedy_accept_scratch_bytes(B, R, V, dtype, splits);
  TRIDA_CHECK(need <= noalloc::kScratchBytes, TRIDA_ERR_WORKSPACE,
              "greedy_accept_noalloc: B=%lld R=%lld V=%lld needs %lld scratch bytes, above the fixed %lld",
              (long long)B, (long long)R, (long long)V, (long long)need, (long long)noalloc::kScratchBytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  const int rc = noalloc_scratch(st, &ws);
  if (rc) return rc;
  return trida_greedy_accept(logits, dtype, B, R, V, batch_stride, row_stride, drafts, K, draft_stride, n_live,
                             ctx_len, argmax_out, n_acc, bonus, crop, ws, noalloc::kScratchBytes, splits, stream);
}

extern "C" int64_t trida_row_argmax_scratch_bytes(int64_t rows, int64_t V, int dtype, int64_t splits) {
  return trida_greedy_accept_scratch_bytes(1, rows, V, dtype, splits);
}

extern "C" int trida_row_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                                int64_t* argmax, float* conf, void* scratch, int64_t scratch_bytes_, int64_t splits,
                                void* stream) {
  TRIDA_CHECK(logits && argmax && scratch, TRIDA_ERR_NULL, "row_argmax: logits, argmax and scratch are required");
  TRIDA_CHECK(rows > 0 && rows <= 65535 && V > 0 && V < INT_MAX && row_stride >= V, TRIDA_ERR_ARG,
              "row_argmax: bad sizes");
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t S;
  float *pval, *psum;
  int* pidx;
  int rc = run_split(logits, dtype, 1, rows, V, 0, row_stride, conf != nullptr, scratch, scratch_bytes_, splits, st,
                     &S, &pval, &pidx, &psum);
  if (rc) return rc;
  hipLaunchKernelGGL(row_finalize_kernel, dim3((unsigned)cdiv(rows, 256)), dim3(256), 0, st, pval, pidx, psum,
                     (int)rows, (int)S, argmax, conf);
  return launch_status("row_argmax/finalize");
}

extern "C" int trida_unmask_top(const int64_t* argmax, const float* conf, int64_t row_stride, uint8_t* masked,
                                int64_t* canvas, int64_t canvas_stride, int64_t B, int64_t block, int64_t count,
                                void* stream) {
  TRIDA_CHECK(argmax && conf && masked && canvas, TRIDA_ERR_NULL, "unmask_top: argmax, conf, masked and canvas are required");
  TRIDA_CHECK(B > 0 && B < INT32_MAX && block >= 1 && block <= kMaxUnmask && count >= 0 && count <= block, TRIDA_ERR_ARG,
              "unmask_top: bad sizes B=%lld block=%lld (<= %d) count=%lld", (long long)B, (long long)block,
              kMaxUnmask, (long long)count);
  TRIDA_CHECK(row_stride >= block && canvas_stride >= block + 1, TRIDA_ERR_ARG, "unmask_top: strides");
  hipLaunchKernelGGL(unmask_top_kernel, dim3((unsigned)B), dim3(256), 0, static_cast<hipStream_t>(stream), argmax, conf,
                     row_stride, masked, canvas, canvas_stride, (int)block, (int)count);
  return launch_status("unmask_top");
}

extern "C" int trida_canvas_advance(const int64_t* argmax, int64_t argmax_stride, const int32_t* n_acc, int64_t* canvas,
                                    int64_t canvas_stride, uint8_t* verify, int32_t* n_keep, int64_t* emit,
                                    int32_t* n_emit, int64_t* committed, int32_t* kind, int64_t B, int64_t N,
                                    int64_t mask_id, void* stream) {
  TRIDA_CHECK(argmax && n_acc && canvas && verify && n_keep && emit && n_emit && committed && kind, TRIDA_ERR_NULL,
              "canvas_advance: every pointer is required");
  TRIDA_CHECK(B > 0 && B < INT32_MAX && N >= 2 && N <= 512, TRIDA_ERR_ARG, "canvas_advance: bad sizes B=%lld N=%lld",
              (long long)B, (long long)N);
  TRIDA_CHECK(argmax_stride >= 2 * N - 1 && canvas_stride >= 2 * N - 1, TRIDA_ERR_ARG, "canvas_advance: strides");
  hipLaunchKernelGGL(canvas_advance_kernel, dim3((unsigned)cdiv(B, 64)), dim3(64), 0, static_cast<hipStream_t>(stream),
                     argmax, argmax_stride, n_acc, canvas, canvas_stride, verify, n_keep, emit, n_emit, committed, kind,
                     (int)B, (int)N, mask_id);
  return launch_status("canvas_advance");
}
