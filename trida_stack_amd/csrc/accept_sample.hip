// Sampled self-spec acceptance (speculative rejection sampling with top-k / top-p truncation).
//
// Three launches on the caller's stream:
//   truncate (grid rows): one 512-thread block per verify row finds the truncated distribution's
//       statistics: m = max y (y = logit / T, the banned id at -inf), thr = the smallest kept y and
//       Zk = sum over kept y of exp(y - m), so that P(x) = [y_x >= thr] exp(y_x - m) / Zk.
//       A sorted, evenly spaced 2048-element sample of the row places a window that should hold the
//       truncation boundary; ONE streaming pass then accumulates the row max, the total mass, the mass
//       above the window, and collects the window's values into LDS, where a bitonic sort and an fp64
//       prefix scan resolve thr exactly. When the window misses (a few heavy tokens outside the
//       sample, massive ties, |y| large enough to overflow the sample-relative exponentials) the block
//       falls back to an exact radix select over the order-preserving keys of y, 8 bits per pass.
//   resid_sums (grid NC x B): every block re-derives its sequence's accepted length from the drafted
//       tokens' ratios P_i(d_i) / q_i(d_i), then sums the correction weights max(0, P_a - q_a) (P_K
//       when every draft is accepted) and P_a over its chunk of the vocabulary, in fp64.
//   resid_pick (grid B): inverse CDF in vocabulary order with one uniform: the chunk where the
//       cumulative weight first exceeds u * total, then the token inside it.
// Nothing allocates; scratch holds the per-row statistics and the chunk sums.
#include <limits.h>
#include <math.h>

#include <algorithm>

#include "common.h"

namespace trida {
namespace {

constexpr int kT = 512;  // threads of the truncation block
constexpr int kTW = kT / kWave;
constexpr int kSample = 2048;
constexpr int kCap = 8192;  // LDS collection capacity (values)
constexpr int kBins = 256;  // digits of one radix pass
constexpr int kMaxTopK = 4096;
constexpr uint32_t kKeyLo = 0x00800000u;  // smallest finite key (key(-inf) + 1)
constexpr uint32_t kKeyHi = 0xff7fffffu;  // largest finite key (key(+inf) - 1)
constexpr int kRT = 256;                  // threads of the residual kernels

// Order-preserving map float -> uint32 (larger value, larger key) and its inverse.
__device__ __forceinline__ uint32_t fkey(float y) {
  const uint32_t u = __float_as_uint(y);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float kval(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// y = logit / T rounded to fp32 exactly as an IEEE fp32 division (the reference divides the fp32
// logits by the temperature), -0 folded into +0 so that equal values have equal keys, the banned id at
// -inf. rt = 1/T in fp64: the fp64 product is within 2^-52 (relative) of x/T, while x/T is never within
// 2^-48 of a midpoint between two floats unless it is one exactly, which needs T's odd significand
// times a 25-bit odd significand to fit 24 bits, i.e. T a power of two, where the product is exact.
// So rounding the fp64 product to fp32 gives the correctly rounded quotient, in three instructions.
template <bool kDiv>
__device__ __forceinline__ float exact_y(float x, double rt) {
  const float y = kDiv ? (float)((double)x * rt) : x;
  return y + 0.f;  // -0 + 0 = +0; every other value is unchanged
}
template <bool kDiv>
__device__ __forceinline__ float make_y(float x, int ix, double rt, int ban) {
  return (ix == ban) ? -INFINITY : exact_y<kDiv>(x, rt);
}

__device__ __forceinline__ int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// ---------------------------------------------------------------- block reductions (512 threads)
__device__ __forceinline__ double block_sum(double v, double* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[threadIdx.x / kWave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kTW; ++w) t += sh[w];
  return t;
}
__device__ __forceinline__ float block_max(float v, double* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[threadIdx.x / kWave] = v;
  __syncthreads();
  float t = -INFINITY;
#pragma unroll
  for (int w = 0; w < kTW; ++w) t = fmaxf(t, (float)sh[w]);
  return t;
}
__device__ __forceinline__ int block_isum(int v, double* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[threadIdx.x / kWave] = (double)v;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < kTW; ++w) t += (int)sh[w];
  return t;
}
// Exclusive prefix sum over the block in thread order; *total gets the block total.
__device__ __forceinline__ double block_excl_scan(double v, double* sh, double* total) {
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  double inc = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const double o = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += o;
  }
  double ex = __shfl_up(inc, 1, kWave);
  if (lane == 0) ex = 0.0;
  __syncthreads();
  if (lane == kWave - 1) sh[w] = inc;
  __syncthreads();
  double base = 0.0, tot = 0.0;
#pragma unroll
  for (int i = 0; i < kTW; ++i) {
    base += (i < w) ? sh[i] : 0.0;
    tot += sh[i];
  }
  *total = tot;
  return base + ex;
}

// Bitonic sort, descending, of s[0..n) (n a power of two); starts and ends with a barrier.
__device__ void sort_desc(float* s, int n) {
  __syncthreads();
  for (int k = 2; k <= n; k <<= 1)
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < (n >> 1); i += kT) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo + j;
        const float a = s[lo], b = s[hi];
        const bool desc = (lo & k) == 0;
        if (desc ? (a < b) : (a > b)) {
          s[lo] = b;
          s[hi] = a;
        }
      }
      __syncthreads();
    }
}

// Appends y (where pred) to s_coll through one LDS counter bump per wave; the counter keeps counting
// past kCap so that an overflow is visible. Called by every lane of the wave.
__device__ __forceinline__ void append(float y, bool pred, float* s_coll, int* s_n) {
  const uint64_t bal = __ballot(pred);
  if (bal == 0) return;
  const int lane = threadIdx.x % kWave;
  int base = 0;
  if (lane == 0) base = atomicAdd(s_n, __popcll(bal));
  base = __shfl(base, 0, kWave);
  const int slot = base + __popcll(bal & ((1ull << lane) - 1ull));
  if (pred && slot < kCap) s_coll[slot] = y;
}

// Calls f(y, ix, valid) for every element of a row; U 16-byte loads in flight per thread.
template <bool kDiv, bool kVec, int U = 4, typename F>
__device__ __forceinline__ void for_each_y(const float* row, int V, double rt, int ban, F&& f) {
  const int tid = threadIdx.x;
  int done = 0;
  if (kVec) {
    const u32x4* row4 = reinterpret_cast<const u32x4*>(row);
    const int n4 = V >> 2;
    for (int base = 0; base < n4; base += kT * U) {
      u32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const u32x4* p = row4 + min(base + u * kT + tid, n4 - 1);
        x[u] = *p;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kT + tid;
        const bool ok = j < n4;
        const float xs[4] = {__uint_as_float(x[u].x), __uint_as_float(x[u].y), __uint_as_float(x[u].z),
                             __uint_as_float(x[u].w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) f(make_y<kDiv>(xs[e], 4 * j + e, rt, ban), 4 * j + e, ok);
      }
    }
    done = n4 << 2;
  }
  for (int base = done; base < V; base += kT) {
    const int ix = base + tid;
    const bool ok = ix < V;
    f(make_y<kDiv>(row[ok ? ix : V - 1], ix, rt, ban), ix, ok);
  }
}

struct TruncArgs {
  const float* logits;
  int64_t batch_stride, row_stride;  // elements
  int R, V;
  double rt;    // 1 / temperature
  int top_k;    // active when 0 < top_k < V
  float top_p;  // active when < 1
  int ban;      // banned id (-1: none)
  int flags;    // bit 0: skip the window pass (exact radix select only)
  int G, first;       // row group: block j of sequence b handles row first + j (rows >= R are skipped)
  const int* state;   // per sequence: -1 = every row so far accepted; >= 0 = decided (skip); null: none
  float* m_out;
  float* thr_out;
  double* zk_out;
  int* status_out;
  int* passes_out;
};

// Value histogram of the streaming pass: 2048 bins of 1/32 nat over d = y - mref in (-24, 40]
// (mref = the sample max); bin 0 holds the largest values. Bin kNB is the spare bin: entries with
// d <= -24, -inf entries, the banned id and padding lanes land there (its mass still counts towards
// the total). d > 40 is caught afterwards from the row max and sends the row to the radix select.
// Each bin is one 64-bit LDS word: the count in bits 46..63 and, below, the sum of r * 2^26 with
// r = exp(d - top of the bin) in (e^-1/32, 1]: one integer LDS atomic per element (fp64 and fp32 LDS
// atomics measured several times slower on gfx950). Rows need V < 2^18 for the count field.
constexpr int kNB = 2048;
constexpr float kTop = 40.f;
constexpr float kPerNat = 32.f;
constexpr double kBinRatio = 0x1.f03f56a88b5d8p-1;  // exp(-1 / kPerNat): the scale of bin b + 1 over bin b
constexpr int kSeg = 4;  // the streaming pass re-places its collection window between segments
constexpr int kCountShift = 46;
constexpr unsigned long long kMassMask = (1ull << kCountShift) - 1ull;
constexpr int kMaxPackedV = (1 << 18) - 1;

// Bin of an element from its raw logit x: t = 32 (40 - d) with d = x / T - mref, as one fma whose
// coefficients the block derives once (tA = -32 / T, tB = 32 (40 + mref)). Monotone in x.
__device__ __forceinline__ unsigned bin_of_t(float t) {
  return min((unsigned)(int)__builtin_amdgcn_fmed3f(t, -1.f, (float)kNB), (unsigned)kNB);
}
// c ? x : y on values: a conditional over two array elements (lvalues) selects their addresses, which
// sends register arrays to scratch memory
__device__ __forceinline__ double pick(bool c, double x, double y) { return c ? x : y; }

// exp(top of the bin) relative to exp(mref); consecutive bins scale by kBinRatio
__device__ __forceinline__ double bin_scale(int bin) { return exp((double)kTop - (double)bin / kPerNat); }
__device__ __forceinline__ double bin_mass(unsigned long long h, double scale) {  // relative to exp(mref)
  return ldexp((double)(h & kMassMask), -26) * scale;
}

struct BinMap {  // the per-row coefficients of the element -> bin / exponent maps
  float tA, tB;  // t = fma(x, tA, tB)
  float rf, nm;  // d = fma(x, rf, nm) = x / T - mref
  __device__ unsigned bin(float x) const { return bin_of_t(fmaf(x, tA, tB)); }
};

struct Shared {
  float coll[kCap];
  unsigned long long hist[kNB + 1];
  unsigned cnt[kBins];  // radix-select digits
  double mass[kBins];
  double red[kTW];
  int n;
  int ipar[4];
  int wlo[kSeg], whi[kSeg];  // the window each segment collected (bins, inclusive)
  int nseg[kSeg];            // collection fill after each segment
  double dpar[4];
  unsigned umax;
};

// Count of j < lim with base + sum_{i<j} e_i < target, e_i = exp(s_i - m) in fp64 (a prefix, since
// the partial sums only grow); *tot = sum_{j<lim} e_j.
__device__ int count_below(const float* s, int lim, double m, double base, double target, double* tot,
                           double* sh) {
  const int L = (lim + kT - 1) / kT;
  const int j0 = min(lim, (int)threadIdx.x * L), j1 = min(lim, j0 + L);
  double loc = 0.0;
  for (int j = j0; j < j1; ++j) loc += exp((double)s[j] - m);
  const double ex = block_excl_scan(loc, sh, tot);
  int c = 0;
  double run = base + ex;
  for (int j = j0; j < j1; ++j) {
    c += run < target;
    run += exp((double)s[j] - m);
  }
  return block_isum(c, sh);
}

// sum over j < n with s_j >= thr of exp(s_j - m)
__device__ __forceinline__ double mass_at_least(const float* s, int n, float thr, double m, double* sh) {
  double loc = 0.0;
  for (int j = threadIdx.x; j < n; j += kT) loc += (s[j] >= thr) ? exp((double)s[j] - m) : 0.0;
  return block_sum(loc, sh);
}

__device__ int count_cmp(const float* s, int n, float v, bool strictly_greater, double* sh) {
  int c = 0;
  for (int j = threadIdx.x; j < n; j += kT) c += strictly_greater ? (s[j] > v) : (s[j] == v);
  return block_isum(c, sh);
}

// Pads the collection to a power of two with -inf and sorts it (descending).
__device__ void sort_collection(Shared& sh, int n) {
  const int np = next_pow2(max(n, 2));
  for (int j = n + threadIdx.x; j < np; j += kT) sh.coll[j] = -INFINITY;
  sort_desc(sh.coll, np);
}

// One fallback pass over the keys: counts/mass (relative to the exact max m) above khi, and either a
// histogram of [klo, khi] in digits of 2^shift keys or a collection of that range. On want_z it also
// sums the whole row's mass and counts its finite entries.
template <bool kDiv, bool kVec, bool kHist>
__device__ void range_pass(const float* row, const TruncArgs& a, float m, uint32_t klo, uint32_t khi, int shift,
                           bool want_z, Shared& sh, int* ca_out, double* ma_out, double* z_out, int* cf_out) {
  if (kHist)
    for (int j = threadIdx.x; j < kBins; j += kT) {
      sh.cnt[j] = 0u;
      sh.mass[j] = 0.0;
    }
  if (threadIdx.x == 0) sh.n = 0;
  __syncthreads();
  int ca = 0, cf = 0;
  double ma = 0.0, z = 0.0;
  for_each_y<kDiv, kVec, 2>(row, a.V, a.rt, a.ban, [&](float y, int ix, bool ok) {
    const bool fin = ok && (y > -INFINITY);
    const uint32_t key = fkey(y);
    const float e = __expf(y - m);
    const bool above = fin && key > khi;
    const bool in = fin && key >= klo && key <= khi;
    ca += above;
    ma += above ? e : 0.f;
    if (want_z) {
      z += fin ? e : 0.f;
      cf += fin;
    }
    if (kHist) {
      if (in) {
        const int bin = (int)((key - klo) >> shift);
        atomicAdd(&sh.cnt[bin], 1u);
        atomicAdd(&sh.mass[bin], (double)e);
      }
    } else {
      append(y, in, sh.coll, &sh.n);
    }
  });
  *ca_out = block_isum(ca, sh.red);
  *ma_out = block_sum(ma, sh.red);
  if (want_z) {
    *z_out = block_sum(z, sh.red);
    *cf_out = block_isum(cf, sh.red);
  }
  __syncthreads();
}

// Exact radix select with the exact row max m. Count mode (use_k): the top_k-th largest value; mass
// mode: the smallest y whose strictly-greater mass is < top_p * Z. Writes thr / Zk (relative to m).
template <bool kDiv, bool kVec>
__device__ void radix_resolve(const float* row, const TruncArgs& a, float m, bool use_k, bool use_p, Shared& sh,
                              float* thr_out, double* zk_out, int* passes) {
  const double md = (double)m;
  uint32_t klo = kKeyLo, khi = kKeyHi;
  int shift = 24;
  int ca = 0, cf = 0;
  double ma = 0.0, Z = 0.0, z = 0.0;
  bool count_mode = use_k;
  const int k = a.top_k;
  double tp = 0.0;
  // results of the select
  float v = -INFINITY;  // count mode: kth; mass mode: thr
  int c_gt = 0, c_eq = 0;
  double zk = 0.0;
  bool resolved = false;
  for (int it = 0; !resolved; ++it) {
    range_pass<kDiv, kVec, true>(row, a, m, klo, khi, shift, it == 0, sh, &ca, &ma, &z, &cf);
    ++*passes;
    if (it == 0) {
      Z = z;
      if (count_mode && cf <= k) count_mode = false;  // fewer finite entries than k: top-k keeps them all
      if (!count_mode && !use_p) {                    // nothing left to select
        *thr_out = -INFINITY;
        *zk_out = Z;
        return;
      }
      tp = (double)a.top_p * Z;
    }
    if (threadIdx.x == 0) {
      const int nb = (int)(((uint64_t)khi - klo) >> shift) + 1;
      double cum = count_mode ? (double)ca : ma;
      int pick = -1, last = -1;
      double cum_last = cum;
      for (int bin = nb - 1; bin >= 0; --bin) {
        if (sh.cnt[bin] == 0u) continue;
        const double add = count_mode ? (double)sh.cnt[bin] : sh.mass[bin];
        if ((count_mode && cum + add >= (double)k) || (!count_mode && cum + add >= tp)) {
          pick = bin;
          break;
        }
        last = bin;
        cum_last = cum;
        cum += add;
      }
      if (pick < 0) {  // mass mode: every entry qualifies, so the smallest one is the threshold
        pick = max(last, 0);
        cum = cum_last;
      }
      sh.ipar[0] = pick;
      sh.dpar[0] = cum;  // count or mass strictly above the picked digit
    }
    __syncthreads();
    const int pick = sh.ipar[0];
    const double cum = sh.dpar[0];
    const uint32_t nlo = klo + ((uint32_t)pick << shift);
    const uint32_t nhi = (uint32_t)min((uint64_t)khi, (uint64_t)nlo + (1ull << shift) - 1ull);
    const unsigned cnt = sh.cnt[pick];
    const double bmass = sh.mass[pick];
    __syncthreads();
    if (nlo == nhi) {  // one key: every entry of the digit has the same value
      v = kval(nlo);
      if (count_mode) {
        c_gt = (int)cum;
        c_eq = (int)cnt;
      } else {
        zk = cum + bmass;
      }
      resolved = true;
    } else if (cnt <= (unsigned)kCap) {
      klo = nlo;
      khi = nhi;
      int ca2 = 0, cf2 = 0;
      double ma2 = 0.0, z2 = 0.0;
      range_pass<kDiv, kVec, false>(row, a, m, klo, khi, 0, false, sh, &ca2, &ma2, &z2, &cf2);
      ++*passes;
      const int n = min(sh.n, kCap);
      sort_collection(sh, n);
      if (count_mode) {
        v = sh.coll[min(max(k - 1 - ca2, 0), max(n - 1, 0))];
        c_gt = ca2 + count_cmp(sh.coll, n, v, true, sh.red);
        c_eq = count_cmp(sh.coll, n, v, false, sh.red);
      } else {
        double tot = 0.0;
        int nk = count_below(sh.coll, n, md, ma2, tp, &tot, sh.red);
        nk = min(max(nk, 1), n);
        v = sh.coll[nk - 1];
        zk = ma2 + mass_at_least(sh.coll, n, v, md, sh.red);
      }
      resolved = true;
    } else {
      klo = nlo;
      khi = nhi;
      shift = shift >= 8 ? shift - 8 : 0;
    }
  }
  if (!count_mode) {
    *thr_out = v;
    *zk_out = zk;
    return;
  }
  // top-k: the values above kth (fewer than k <= kMaxTopK, so they fit), then the nucleus over the
  // k-value list {values > kth} + (k - c_gt) copies of kth
  const float kth = v;
  int ca2 = 0, cf2 = 0;
  double ma2 = 0.0, z2 = 0.0;
  const uint32_t kk = fkey(kth);
  range_pass<kDiv, kVec, false>(row, a, m, kk + 1u, kKeyHi, 0, false, sh, &ca2, &ma2, &z2, &cf2);
  ++*passes;
  const int n = min(sh.n, kCap);
  sort_collection(sh, n);
  const double e_k = exp((double)kth - md);
  double s_gt = 0.0;
  const double copies = (double)(k - c_gt);
  if (use_p) {
    double tot = 0.0;
    // total first: S = sum_{coll} e + copies * e_k
    (void)count_below(sh.coll, n, md, 0.0, -1.0, &tot, sh.red);
    s_gt = tot;
    const double target = (double)a.top_p * (s_gt + copies * e_k);
    int nk = count_below(sh.coll, n, md, 0.0, target, &tot, sh.red);
    int ncp = 0;
    for (int i = threadIdx.x; i < k - c_gt; i += kT) ncp += (s_gt + (double)i * e_k) < target;
    ncp = block_isum(ncp, sh.red);
    nk = max(nk + ncp, 1);
    if (nk <= c_gt) {
      const float thr = sh.coll[nk - 1];
      *thr_out = thr;
      *zk_out = mass_at_least(sh.coll, n, thr, md, sh.red);
      return;
    }
  } else {
    double tot = 0.0;
    (void)count_below(sh.coll, n, md, 0.0, -1.0, &tot, sh.red);
    s_gt = tot;
  }
  *thr_out = kth;
  *zk_out = s_gt + (double)c_eq * e_k;
}

// Keeps the collected logits whose bin lies in [lo, hi] and that came from a segment in the bit set
// `segs` (entry j came from segment s when nseg[s-1] <= j < nseg[s]), packed at the front of
// sh.coll; returns how many.
__device__ __forceinline__ int compact_bins(Shared& sh, const BinMap& bm, int n, int lo, int hi, unsigned segs) {
  constexpr int kPer = kCap / kT;
  float v[kPer];
  bool kp[kPer];
  int keep = 0;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int j = (int)threadIdx.x * kPer + u;
    v[u] = j < n ? sh.coll[j] : -INFINITY;
    const int bin = (int)bm.bin(v[u]);
    int s = 0;
    while (s < kSeg - 1 && j >= sh.nseg[s]) ++s;
    kp[u] = (j < n) && bin >= lo && bin <= hi && ((segs >> s) & 1u);
    keep += kp[u];
  }
  double tot = 0.0;
  int w = (int)block_excl_scan((double)keep, sh.red, &tot);  // every read of sh.coll precedes its barriers
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (kp[u]) sh.coll[w++] = v[u];
  __syncthreads();
  return (int)tot;
}

// Appends the values of xv whose bit is set in mask. Called by every lane of the wave: the lanes'
// offsets are the wave-exclusive prefix of their counts, summed from the counts' bit planes (a ballot
// and a masked bit count each), and one LDS counter bump per wave takes the wave's total (same-address
// LDS atomics serialise, one lane after another).
template <int N>
__device__ __forceinline__ void append_batch(const float (&xv)[N], unsigned mask, Shared& sh) {
  constexpr int kPlanes = N >= 16 ? 5 : N >= 8 ? 4 : N >= 4 ? 3 : N >= 2 ? 2 : 1;  // bits of a count <= N
  const int c = __popc(mask);
  int pre = 0, tot = 0;
#pragma unroll
  for (int bit = 0; bit < kPlanes; ++bit) {
    const uint64_t bb = __ballot((c >> bit) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bb, 0u)) << bit;
    tot += __popcll(bb) << bit;
  }
  if (tot == 0) return;  // wave-uniform
  int base = 0;
  if (threadIdx.x % kWave == 0) base = atomicAdd(&sh.n, tot);
  int pos = __builtin_amdgcn_readfirstlane(base) + pre;
#pragma unroll
  for (int e = 0; e < N; ++e)
    if ((mask >> e) & 1u) {
      if (pos < kCap) sh.coll[pos] = xv[e];
      ++pos;
    }
}

// Streams the row's elements [e0, e1) (e0 and e1 multiples of 4 on the vector path, except e1 = V),
// in the logits' own units: the division by the temperature is folded into the bin / exponent maps,
// and the exact y = x / T is only formed for the few collected values.
// kHist: histogram every element, track the max and the NaN flag, collect the bins [wlo, whi].
// Otherwise only collect the bins [wlo, whi]. The element body is branch-free; the banned id and the
// padding lanes of a last partial tile take a separate path for that tile only.
template <bool kVec, bool kHist>
__device__ void stream_segment(const float* row, const TruncArgs& a, const BinMap& bm, int e0, int e1, int wlo,
                               int whi, Shared& sh, float& mx, unsigned& nanbits) {
  constexpr int U = 4;
  const int tid = threadIdx.x;
  const unsigned wspan = (unsigned)(whi - wlo);
  auto one = [&](float x, unsigned& mask, int e) {
    const unsigned bin = bm.bin(x);
    if (kHist) {
      const float d = fmaf(x, bm.rf, bm.nm);
      const float top = fmaf((float)bin, -1.f / kPerNat, kTop);
      const float r = __builtin_amdgcn_exp2f(fmaf(d - top, 1.44269504f, 26.f));  // r * 2^26
      atomicAdd(&sh.hist[bin], (1ull << kCountShift) | (unsigned long long)(unsigned)r);
      mx = fmaxf(mx, x);
      nanbits = max(nanbits, __float_as_uint(x) << 1);  // a NaN sorts above +-inf here
    }
    mask |= (unsigned)((unsigned)((int)bin - wlo) <= wspan) << e;
  };
  int t0 = e0;
  if (kVec) {
    const u32x4* row4 = reinterpret_cast<const u32x4*>(row);
    const int v0 = e0 >> 2, v1 = (e1 == a.V) ? (a.V >> 2) : (e1 >> 2);
    const int vb = a.ban >= 0 ? (a.ban >> 2) : -1;
    // the next tile's loads are issued before the current tile is folded, so the fold hides their
    // latency; addresses are clamped to the last vector (the last tile's prefetch reads one line)
    auto load = [&](u32x4 (&dst)[U], int base) {
#pragma unroll
      for (int u = 0; u < U; ++u) dst[u] = row4[min(base + u * kT + tid, v1 - 1)];
    };
    u32x4 xn[U];
    if (v0 < v1) load(xn, v0);
    for (int base = v0; base < v1; base += kT * U) {
      u32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = xn[u];
      load(xn, base + kT * U);
      float xv[4 * U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        xv[4 * u + 0] = __uint_as_float(x[u].x);
        xv[4 * u + 1] = __uint_as_float(x[u].y);
        xv[4 * u + 2] = __uint_as_float(x[u].z);
        xv[4 * u + 3] = __uint_as_float(x[u].w);
      }
      // wave-uniform: does this tile hold the banned id or padding lanes?
      if (base + kT * U > v1 || (unsigned)(vb - base) < (unsigned)(kT * U)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = base + u * kT + tid;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (j >= v1 || 4 * j + e == a.ban) xv[4 * u + e] = -INFINITY;
        }
      }
      unsigned mask = 0u;
#pragma unroll
      for (int e = 0; e < 4 * U; ++e) one(xv[e], mask, e);
      append_batch(xv, mask, sh);
    }
    t0 = max(e0, v1 << 2);
  }
  for (int base = t0; base < e1; base += kT) {
    const int ix = base + tid;
    float xv[1];
    xv[0] = (ix < e1 && ix != a.ban) ? row[ix < e1 ? ix : e1 - 1] : -INFINITY;
    unsigned mask = 0u;
    one(xv[0], mask, 0);
    append_batch(xv, mask, sh);
  }
}

// Element bounds of segment s of the streaming pass.
template <bool kVec>
__device__ __forceinline__ void seg_bounds(int V, int s, int* e0, int* e1) {
  if (kVec) {
    const int n4 = V >> 2;
    *e0 = 4 * (int)((int64_t)n4 * s / kSeg);
    *e1 = s == kSeg - 1 ? V : 4 * (int)((int64_t)n4 * (s + 1) / kSeg);
  } else {
    *e0 = (int)((int64_t)V * s / kSeg);
    *e1 = (int)((int64_t)V * (s + 1) / kSeg);
  }
}

// Places a collection window from a histogram of part of the row (the sample, or the segments seen
// so far): the bin where that histogram's own boundary falls (the k_seen-th largest for top-k, the
// top_p mass point for top-p), widened to about `budget` entries of the next segment; `scale` =
// entries of the next segment per counted entry.
__device__ void place_window(Shared& sh, bool use_k, float top_p, double k_seen, double scale, double budget,
                             int* wlo, int* whi) {
  constexpr int kBPT = kNB / kT;
  const int tid = threadIdx.x;
  double lm = 0.0, lc = 0.0;
  double bm[kBPT], bc[kBPT];
  double sc = bin_scale(tid * kBPT);
#pragma unroll
  for (int u = 0; u < kBPT; ++u) {
    const unsigned long long h = sh.hist[tid * kBPT + u];
    bc[u] = (double)(h >> kCountShift);
    bm[u] = (double)(float)bin_mass(h, sc);
    sc *= kBinRatio;
    lm += bm[u];
    lc += bc[u];
  }
  double zb = 0.0, cbins = 0.0;
  const double exm = block_excl_scan(lm, sh.red, &zb);
  const double exc = block_excl_scan(lc, sh.red, &cbins);
  if (tid == 0) {
    sh.ipar[0] = INT_MAX;
    sh.ipar[1] = INT_MAX;
    sh.ipar[2] = -1;
  }
  __syncthreads();
  const double tgt = use_k ? k_seen : (double)top_p * (zb + bin_mass(sh.hist[kNB], bin_scale(kNB)));
  double run = use_k ? exc : exm;
#pragma unroll
  for (int u = 0; u < kBPT; ++u) {
    const double add = pick(use_k, bc[u], bm[u]);
    if (run < tgt && run + add >= tgt) atomicMin(&sh.ipar[0], tid * kBPT + u);
    run += add;
  }
  __syncthreads();
  int B = sh.ipar[0];
  if (B == INT_MAX) B = kNB - 1;
  if (tid == B / kBPT) {
    double c = exc;
#pragma unroll
    for (int u = 0; u < kBPT; ++u) c += u < B % kBPT ? bc[u] : 0.0;  // unrolled: bc stays in registers
    sh.dpar[1] = c;                                                 // count above B
    sh.dpar[2] = (double)(sh.hist[B] >> kCountShift);                // count in B
  }
  __syncthreads();
  const double cB = sh.dpar[1], nB = sh.dpar[2];
  const double half = budget / scale / 2.0;  // in counted entries
  const double lo_c = use_k ? -1.0 : cB - half, hi_c = use_k ? budget / scale : cB + nB + half;
  // the first bin whose cumulative count passes lo_c and the last one that starts below hi_c: the
  // cumulative count (exact in fp64) only grows with the bin, so one bin of each test sees the
  // transition and a single atomic per test lands (same-address LDS atomics serialise)
  double c = exc;
#pragma unroll
  for (int u = 0; u < kBPT; ++u) {
    const int bin = tid * kBPT + u;
    if (c + bc[u] > lo_c && (bin == 0 || c <= lo_c)) atomicMin(&sh.ipar[1], bin);
    if (c < hi_c && (bin == kNB - 1 || c + bc[u] >= hi_c)) atomicMax(&sh.ipar[2], bin);
    c += bc[u];
  }
  __syncthreads();
  *wlo = use_k ? 0 : min(sh.ipar[1], B);
  *whi = min(max(sh.ipar[2], B) + 1, kNB - 1);  // one bin of slack below: values tied across a bin edge
  __syncthreads();
}

// Exact y = x / T of the collected logits, in place.
template <bool kDiv>
__device__ void collected_to_y(Shared& sh, int n, double rt) {
  for (int j = threadIdx.x; j < n; j += kT) sh.coll[j] = exact_y<kDiv>(sh.coll[j], rt);
  __syncthreads();
}

// Top-p candidates (the collected logits of the boundary bin B and of bin B + 1) to exact y, in place,
// packed at the front; returns how many. Bins are monotone in the logit, so a value of bin B + 1 is
// <= every value of bin B in y and can only be kept when it ties with the smallest of them: the
// others are dropped, which about halves what is sorted.
template <bool kDiv>
__device__ int boundary_to_y(Shared& sh, const BinMap& bm, int n, int B, double rt) {
  constexpr int kPer = kCap / kT;
  float y[kPer];
  unsigned inb = 0u;  // bit u: entry u is in bin B (then: is kept)
  float ymin = INFINITY;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int j = (int)threadIdx.x * kPer + u;
    const float x = j < n ? sh.coll[j] : -INFINITY;
    const bool in = j < n && (int)bm.bin(x) == B;
    y[u] = j < n ? exact_y<kDiv>(x, rt) : -INFINITY;
    ymin = in ? fminf(ymin, y[u]) : ymin;
    inb |= (unsigned)in << u;
  }
  ymin = -block_max(-ymin, sh.red);
  const int nl = max(min(n - (int)threadIdx.x * kPer, kPer), 0);  // this thread's entries
#pragma unroll
  for (int u = 0; u < kPer; ++u) inb |= (unsigned)(u < nl && y[u] == ymin) << u;
  double tot = 0.0;
  int w = (int)block_excl_scan((double)__popc(inb), sh.red, &tot);  // every read of sh.coll precedes its barriers
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if ((inb >> u) & 1u) sh.coll[w++] = y[u];
  __syncthreads();
  return (int)tot;
}

template <bool kDiv, bool kVec>
__global__ __launch_bounds__(kT, 4) void truncate_kernel(TruncArgs a) {
  __shared__ Shared sh;
  const int b = blockIdx.x / a.G, i = a.first + (int)(blockIdx.x % a.G);
  if (i >= a.R || (a.state && a.state[b] >= 0)) return;  // block-uniform: past the rows, or decided
  const int r = b * a.R + i;
  const float* row = a.logits + (int64_t)b * a.batch_stride + (int64_t)i * a.row_stride;
  const int V = a.V, tid = threadIdx.x;
  const bool use_k = a.top_k > 0 && a.top_k < V;
  const bool use_p = a.top_p < 1.f;
  const bool collect = use_k || use_p;
  const bool window = !(a.flags & 1) && V <= kMaxPackedV;
  int passes = 0;  // segments streamed (kSeg = one pass over the row)

  float mx = -INFINITY;  // max logit (the banned id excluded)
  unsigned nanbits = 0u;
  float mref = 0.f;
  BinMap bm{};
  if (window) {
    // ---- sample: evenly spaced entries; their max is the exponent reference of the pass, their
    // histogram places the first segment's window
    const int ns = min(kSample, V);
    float xs[kSample / kT];
    float smax = -INFINITY;
    if (kVec && V >= 4 * kSample) {
      // kT evenly spaced 16-byte vectors of 4 adjacent entries each: a line per 4 entries (entries one
      // by one would fetch a line each, a quarter of the row's bytes at V = 248320)
      static_assert(kSample == 4 * kT, "one vector of the sample per thread");
      const int jv = (int)((int64_t)tid * (V >> 2) / kT);
      const u32x4 w = reinterpret_cast<const u32x4*>(row)[jv];
      const float x4[4] = {__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w)};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        xs[u] = (4 * jv + u != a.ban && x4[u] == x4[u]) ? x4[u] : -INFINITY;
        smax = xs[u] < INFINITY ? fmaxf(smax, xs[u]) : smax;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kSample / kT; ++u) {
        const int j = u * kT + tid;
        const int ix = (int)((int64_t)min(j, ns - 1) * V / ns);
        const float x = row[ix];
        xs[u] = (j < ns && ix != a.ban && x == x) ? x : -INFINITY;
        smax = xs[u] < INFINITY ? fmaxf(smax, xs[u]) : smax;
      }
    }
    smax = block_max(smax, sh.red);
    mref = smax > -INFINITY ? exact_y<kDiv>(smax, a.rt) : 0.f;
    const float rf = (float)a.rt;
    bm.tA = -kPerNat * rf;
    bm.tB = kPerNat * (kTop + mref);
    bm.rf = rf;
    bm.nm = -mref;
    for (int j = tid; j <= kNB; j += kT) sh.hist[j] = 0ull;
    __syncthreads();
    int w_lo = kNB + 1, w_hi = kNB + 1;  // empty
    if (collect) {
#pragma unroll
      for (int u = 0; u < kSample / kT; ++u) {
        const float x = xs[u] < INFINITY ? xs[u] : -INFINITY;
        const unsigned bin = bm.bin(x);
        const float d = fmaf(x, bm.rf, bm.nm);
        const float top = fmaf((float)bin, -1.f / kPerNat, kTop);
        const float rr = __builtin_amdgcn_exp2f(fmaf(d - top, 1.44269504f, 26.f));
        atomicAdd(&sh.hist[bin], (1ull << kCountShift) | (unsigned long long)(unsigned)rr);
      }
      __syncthreads();
      int s0, s1;
      seg_bounds<kVec>(V, 0, &s0, &s1);
      place_window(sh, use_k, a.top_p, (double)a.top_k * ns / V, (double)(s1 - s0) / ns, 0.2 * kCap, &w_lo, &w_hi);
      for (int j = tid; j <= kNB; j += kT) sh.hist[j] = 0ull;
    }
    if (tid == 0) sh.n = 0;
    __syncthreads();

    // ---- the streaming pass, kSeg segments: max, histogram, collection of a window re-placed from the
    // exact histogram after every segment
    for (int s = 0; s < kSeg; ++s) {
      int e0, e1;
      seg_bounds<kVec>(V, s, &e0, &e1);
      if (tid == 0) {
        sh.wlo[s] = w_lo;
        sh.whi[s] = w_hi;
      }
      stream_segment<kVec, true>(row, a, bm, e0, e1, w_lo, w_hi, sh, mx, nanbits);
      ++passes;
      __syncthreads();
      if (tid == 0) sh.nseg[s] = sh.n;
      if (collect && s + 1 < kSeg) {
        __syncthreads();
        int n0, n1;
        seg_bounds<kVec>(V, s + 1, &n0, &n1);
        const double seen = (double)e1, next = (double)(n1 - n0);
        const double room = max(0.6 * kCap - (double)min(sh.n, kCap), 0.0);
        place_window(sh, use_k, a.top_p, (double)a.top_k * seen / V, next / seen, room / (kSeg - 1 - s), &w_lo,
                     &w_hi);
      }
    }
  } else {
    for_each_y<kDiv, kVec>(row, V, a.rt, a.ban, [&](float y, int ix, bool ok) {
      mx = fmaxf(mx, ok ? y : -INFINITY);
      nanbits = max(nanbits, ok ? __float_as_uint(y) << 1 : 0u);
    });
    passes += kSeg;
  }
  mx = block_max(mx, sh.red);
  if (tid == 0) sh.umax = 0u;
  __syncthreads();
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) nanbits = max(nanbits, (unsigned)__shfl_xor((int)nanbits, off, kWave));
  if (tid % kWave == 0) atomicMax(&sh.umax, nanbits);  // one atomic per wave
  __syncthreads();
  const bool bad = sh.umax > 0xff000000u || mx == INFINITY;  // a NaN, or a +inf logit
  // the exact row max of y (the window path tracked the raw logits; y = x / T is monotone in x)
  const float ymax = window ? exact_y<kDiv>(mx, a.rt) : mx;
  float thr = -INFINITY;
  double zk = 0.0;
  int status = 0;
  if (bad) {
    status = 1;
  } else if (!(ymax > -INFINITY)) {
    status = 2;
  } else {
    bool ok = window && !(ymax - mref > kTop);
    const int n = sh.n;
    const double md = (double)ymax;
    const double scale = exp((double)mref - md);
    if (ok) {
      // each thread owns kNB / kT consecutive bins; exclusive scans give the mass / count above each
      constexpr int kBPT = kNB / kT;
      double lm = 0.0, lc = 0.0;
      double bms[kBPT], bcs[kBPT];
      double sc = bin_scale(tid * kBPT);
#pragma unroll
      for (int u = 0; u < kBPT; ++u) {
        const unsigned long long h = sh.hist[tid * kBPT + u];
        bcs[u] = (double)(h >> kCountShift);
        bms[u] = bin_mass(h, sc);
        sc *= kBinRatio;
        lm += bms[u];
        lc += bcs[u];
      }
      double zb = 0.0, cbins = 0.0;
      const double exm = block_excl_scan(lm, sh.red, &zb);
      const double exc = block_excl_scan(lc, sh.red, &cbins);
      const double Z = zb + bin_mass(sh.hist[kNB], bin_scale(kNB));
      if (!collect) {
        zk = Z * scale;
      } else {
        // the bin holding the k-th largest value (top-k) or the nucleus boundary (top-p)
        const double tgt = use_k ? (double)a.top_k : (double)a.top_p * Z;
        if (tid == 0) sh.ipar[0] = INT_MAX;
        __syncthreads();
        double run = use_k ? exc : exm;
#pragma unroll
        for (int u = 0; u < kBPT; ++u) {
          const double add = pick(use_k, bcs[u], bms[u]);
          if (run < tgt && run + add >= tgt) atomicMin(&sh.ipar[0], tid * kBPT + u);
          run += add;
        }
        __syncthreads();
        const int B = sh.ipar[0];
        if (B != INT_MAX && tid == B / kBPT) {  // the owner publishes the count / mass above the bin
          double cum = use_k ? exc : exm;
#pragma unroll
          for (int u = 0; u < kBPT; ++u) cum += u < B % kBPT ? pick(use_k, bcs[u], bms[u]) : 0.0;
          sh.dpar[0] = cum;
        }
        __syncthreads();
        if (B == INT_MAX) {
          ok = false;  // the target lies below the histogram's range
        } else {
          // values tied in y may straddle a bin edge (the bins come from the logits), so the
          // candidate set takes one more bin below the boundary bin
          const double cum = sh.dpar[0];
          const int c_lo = use_k ? 0 : B, c_hi = min(B + 1, kNB - 1);
          double need = use_k ? cum : 0.0;
          for (int bb = B; bb <= c_hi; ++bb) need += (double)(sh.hist[bb] >> kCountShift);
          if (need > kCap) {
            ok = false;
          } else {
            // keep what the segments whose window held [c_lo, c_hi] collected (and that fit the
            // collection); stream the others again
            unsigned complete = 0u;
            for (int s = 0; s < kSeg; ++s)
              complete |= (unsigned)(c_lo >= sh.wlo[s] && c_hi <= sh.whi[s] && sh.nseg[s] <= kCap) << s;
            int n2 = compact_bins(sh, bm, min(n, kCap), c_lo, c_hi, complete);
            __syncthreads();
            if (tid == 0) sh.n = n2;
            __syncthreads();
            for (int s = 0; s < kSeg; ++s) {
              if ((complete >> s) & 1u) continue;
              int e0, e1;
              seg_bounds<kVec>(V, s, &e0, &e1);
              stream_segment<kVec, false>(row, a, bm, e0, e1, c_lo, c_hi, sh, mx, nanbits);
              ++passes;
            }
            __syncthreads();
            n2 = min(sh.n, kCap);
            if (use_k)
              collected_to_y<kDiv>(sh, n2, a.rt);
            else
              n2 = boundary_to_y<kDiv>(sh, bm, n2, B, a.rt);
            sort_collection(sh, n2);
            if (use_k) {
              const int k = min(a.top_k, n2);
              thr = sh.coll[k - 1];
              if (use_p) {
                double Sk = 0.0, tot = 0.0;
                (void)count_below(sh.coll, k, md, 0.0, -1.0, &Sk, sh.red);
                const int nk = max(count_below(sh.coll, k, md, 0.0, (double)a.top_p * Sk, &tot, sh.red), 1);
                thr = sh.coll[nk - 1];
              }
              zk = mass_at_least(sh.coll, n2, thr, md, sh.red);
            } else {
              const double base = cum * scale, target = tgt * scale;
              double tot = 0.0;
              const int nk = min(max(count_below(sh.coll, n2, md, base, target, &tot, sh.red), 1), max(n2, 1));
              thr = sh.coll[nk - 1];
              zk = base + mass_at_least(sh.coll, n2, thr, md, sh.red);
            }
          }
        }
      }
    }
    if (!ok) {
      int rp = 0;
      radix_resolve<kDiv, kVec>(row, a, ymax, use_k, use_p, sh, &thr, &zk, &rp);
      passes += rp * kSeg;
    }
  }
  if (tid == 0) {
    a.m_out[r] = ymax;
    a.thr_out[r] = thr;
    a.zk_out[r] = zk;
    a.status_out[r] = status;
    if (a.passes_out) a.passes_out[r] = passes;
  }
}

// ---------------------------------------------------------------- acceptance and correction
struct AcceptArgs {
  const float* p;
  int64_t p_bs, p_rs;
  const float* q;
  int64_t q_bs, q_rs;
  const int64_t* drafts;
  int64_t d_st;
  const int32_t* n_live;
  const float* u_acc;
  int64_t u_st;
  const float* u_samp;
  const int64_t* ctx;
  int B, V, K;
  double rt;  // 1 / temperature
  int ban;
  const float* m;  // [B * (K + 1)] row statistics
  const float* thr;
  const double* zk;
  const int* status;
  int* state;    // per sequence: -1 while every verified draft was accepted, else the accepted length
  int* rstatus;  // per sequence: OR of the row statuses seen
  int NC, chunk;
  double* sums;  // [B][NC][2]: correction weight, P
  int32_t* n_acc;
  int64_t* token;
  int64_t* crop;
  double* ratio;  // [B, K] or null
  int32_t* status_out;
};

// P_row(x) exactly (fp64 exponential) from the row statistics, 0 outside the kept set: the drafted
// tokens' probabilities in the accept test.
__device__ __forceinline__ double prob_exact(const AcceptArgs& a, int srow, float x, int ix) {
  const float y = make_y<true>(x, ix, a.rt, a.ban);  // the product with rt = 1 is exact
  if (!(y > -INFINITY) || !(y >= a.thr[srow])) return 0.0;
  return exp((double)y - (double)a.m[srow]) / a.zk[srow];
}

// The correction draw's weights over a row (fp32 exponential: a relative error of ~1e-7 per entry,
// so the cumulative weight is off by at most ~1e-7 in probability units).
struct RowW {
  const float* p;
  const float* q;  // null: weights are P_K itself
  float m, thr, inv_zk;
  double rt;
  int ban;
  __device__ __forceinline__ void at(int ix, float* w, float* pp) const {
    const float y = make_y<true>(p[ix], ix, rt, ban);
    const float P = (y > -INFINITY && y >= thr) ? __expf(y - m) * inv_zk : 0.f;
    *pp = P;
    *w = q ? fmaxf(P - q[ix], 0.f) : P;
  }
};
__device__ __forceinline__ RowW row_weights(const AcceptArgs& a, int b, int r) {
  const int srow = b * (a.K + 1) + r;
  RowW w;
  w.p = a.p + (int64_t)b * a.p_bs + (int64_t)r * a.p_rs;
  w.q = r < a.K ? a.q + (int64_t)b * a.q_bs + (int64_t)r * a.q_rs : nullptr;
  w.m = a.m[srow];
  w.thr = a.thr[srow];
  w.inv_zk = (float)(1.0 / a.zk[srow]);
  w.rt = a.rt;
  w.ban = a.ban;
  return w;
}

__device__ __forceinline__ double rblock_sum(double v, double* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[threadIdx.x / kWave] = v;
  __syncthreads();
  double t = 0.0;
#pragma unroll
  for (int w = 0; w < kRT / kWave; ++w) t += sh[w];
  return t;
}

// The accept test of the row group [first, first + G) of sequence b, one wave: the drafted token's
// ratio P_i(d_i) / q_i(d_i) per row, accepted while ratio >= 1 or u_i < ratio (and i < n_live). Decides
// the sequence at its first rejection, or once row K (the bonus row) has been reached.
__global__ __launch_bounds__(kWave) void accept_scan_kernel(AcceptArgs a, int first, int G) {
  const int b = blockIdx.x, lane = threadIdx.x;
  if (first > 0 && a.state[b] >= 0) return;
  const int i = first + lane;
  const bool row_here = lane < G && i <= a.K;
  const bool draft_here = lane < G && i < a.K;
  const int live = a.n_live ? min(max((int)a.n_live[b], 0), a.K) : a.K;
  bool acc = false;
  double ratio = 0.0;
  if (draft_here) {
    const int64_t d = a.drafts[(int64_t)b * a.d_st + i];
    if (d >= 0 && d < a.V) {
      const int srow = b * (a.K + 1) + i;
      const double P = prob_exact(a, srow, a.p[(int64_t)b * a.p_bs + (int64_t)i * a.p_rs + d], (int)d);
      const double q = (double)a.q[(int64_t)b * a.q_bs + (int64_t)i * a.q_rs + d];
      ratio = q > 0.0 ? P / fmax(q, 1e-30) : 0.0;
      acc = (i < live) && (ratio >= 1.0 || (double)a.u_acc[(int64_t)b * a.u_st + i] < ratio);
    }
  }
  const uint64_t drafts = __ballot(draft_here);
  const uint64_t rej = drafts & ~__ballot(acc);
  int n = -1;  // still open
  if (rej) n = first + __builtin_ctzll(rej);
  else if (first + G > a.K) n = a.K;  // this group holds row K: every draft accepted
  int st = row_here ? a.status[b * (a.K + 1) + i] : 0;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) st |= __shfl_xor(st, off, kWave);
  if (a.ratio && draft_here && (n < 0 || i <= n)) a.ratio[(int64_t)b * a.K + i] = ratio;
  if (lane == 0) {
    a.state[b] = n;
    a.rstatus[b] = (first > 0 ? a.rstatus[b] : 0) | st;
  }
}

__global__ __launch_bounds__(kRT) void resid_sums_kernel(AcceptArgs a) {
  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x;
  __shared__ int s_nacc;
  __shared__ double s_red[kRT / kWave];
  if (tid == 0) s_nacc = min(max(a.state[b], 0), a.K);
  __syncthreads();
  if (c == 0) {  // the per-sequence outputs; ratios past the first rejection are 0
    const int n_acc = s_nacc;
    if (a.ratio)
      for (int i = n_acc + 1 + tid; i < a.K; i += kRT) a.ratio[(int64_t)b * a.K + i] = 0.0;
    if (tid == 0) {
      a.n_acc[b] = n_acc;
      a.crop[b] = (a.ctx ? a.ctx[b] : 0) + 1 + n_acc;
      a.status_out[b] = a.rstatus[b];
    }
  }
  __syncthreads();
  const RowW rw = row_weights(a, b, s_nacc);
  const int lo = c * a.chunk, hi = min(a.V, lo + a.chunk);
  double sw = 0.0, sp = 0.0;
  for (int ix = lo + tid; ix < hi; ix += kRT) {
    float w, pp;
    rw.at(ix, &w, &pp);
    sw += w;
    sp += pp;
  }
  sw = rblock_sum(sw, s_red);
  sp = rblock_sum(sp, s_red);
  if (tid == 0) {
    a.sums[((int64_t)b * a.NC + c) * 2 + 0] = sw;
    a.sums[((int64_t)b * a.NC + c) * 2 + 1] = sp;
  }
}

constexpr int kPickChunk = 4096;  // the largest chunk: its weights fit the pick kernel's LDS

__global__ __launch_bounds__(kRT) void resid_pick_kernel(AcceptArgs a) {
  const int b = blockIdx.x, tid = threadIdx.x;
  const int lane = tid % kWave, w = tid / kWave;
  __shared__ int s_chunk, s_last, s_tok, s_sel;
  __shared__ double s_t;
  __shared__ double s_red[kRT / kWave];
  __shared__ float s_w[kPickChunk];
  const int r = a.n_acc[b];
  if (tid == 0) {
    const double* s = a.sums + (int64_t)b * a.NC * 2;
    double tw = 0.0, tp = 0.0;
    for (int c = 0; c < a.NC; ++c) {
      tw += s[2 * c];
      tp += s[2 * c + 1];
    }
    const int sel = tw > 0.0 ? 0 : 1;  // an empty residual draws from P itself
    const double total = sel ? tp : tw;
    const double t = (double)a.u_samp[b] * total;
    double cum = 0.0;
    int pick = -1, lastpos = -1;
    for (int c = 0; c < a.NC; ++c) {
      const double v = s[2 * c + sel];
      if (v > 0.0) lastpos = c;
      if (pick < 0 && cum + v > t) {
        pick = c;
        break;
      }
      cum += v;
    }
    s_last = pick < 0;
    s_chunk = pick < 0 ? max(lastpos, 0) : pick;
    s_t = t - cum;
    s_tok = INT_MAX;
    s_sel = sel;
  }
  __syncthreads();
  const int c = s_chunk, sel = s_sel;
  const bool last = s_last;
  const double t = s_t;
  const int lo = c * a.chunk, hi = min(a.V, lo + a.chunk), len = hi - lo;
  // stage the chunk's weights in LDS with coalesced loads, then scan contiguous runs per thread
  const RowW rw = row_weights(a, b, r);
  for (int j = tid; j < len; j += kRT) {
    float wt, pp;
    rw.at(lo + j, &wt, &pp);
    s_w[j] = sel ? pp : wt;
  }
  __syncthreads();
  const int L = (len + kRT - 1) / kRT;
  const int j0 = min(len, tid * L), j1 = min(len, j0 + L);
  double loc = 0.0;
  int lastpos = -1;
  for (int j = j0; j < j1; ++j) {
    loc += (double)s_w[j];
    if (s_w[j] > 0.f) lastpos = lo + j;
  }
  // exclusive scan over the block (thread order = vocabulary order)
  double inc = loc;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const double o = __shfl_up(inc, off, kWave);
    if (lane >= off) inc += o;
  }
  double ex = __shfl_up(inc, 1, kWave);
  if (lane == 0) ex = 0.0;
  if (lane == kWave - 1) s_red[w] = inc;
  __syncthreads();
  for (int i = 0; i < w; ++i) ex += s_red[i];
  int found = INT_MAX;
  if (!last && ex <= t && t < ex + loc) {
    double run = ex;
    for (int j = j0; j < j1; ++j) {
      run += (double)s_w[j];
      if (run > t) {
        found = lo + j;
        break;
      }
    }
  }
  if (found != INT_MAX) atomicMin(&s_tok, found);
  // the last positive-weight token of the chunk: used when u * total lands past the summed weight
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lastpos = max(lastpos, __shfl_xor(lastpos, off, kWave));
  __syncthreads();
  if (lane == 0) s_red[w] = (double)lastpos;
  __syncthreads();
  if (tid == 0) {
    int lp = -1;
    for (int i = 0; i < kRT / kWave; ++i) lp = max(lp, (int)s_red[i]);
    const int tok = s_tok != INT_MAX ? s_tok : max(lp, 0);
    a.token[b] = tok;
  }
}

int ban_of(int64_t ban_id, int64_t V) { return (ban_id >= 0 && ban_id < V) ? (int)ban_id : -1; }

bool vec_ok(const void* p, int64_t V, int64_t bs, int64_t rs) {
  return ((uintptr_t)p % 16 == 0) && V % 4 == 0 && bs % 4 == 0 && rs % 4 == 0;
}

int launch_truncate(const TruncArgs& ta, int rows, bool vec, hipStream_t st) {
  const bool div = ta.rt != 1.0;
  if (div && vec) hipLaunchKernelGGL((truncate_kernel<true, true>), dim3(rows), dim3(kT), 0, st, ta);
  else if (div) hipLaunchKernelGGL((truncate_kernel<true, false>), dim3(rows), dim3(kT), 0, st, ta);
  else if (vec) hipLaunchKernelGGL((truncate_kernel<false, true>), dim3(rows), dim3(kT), 0, st, ta);
  else hipLaunchKernelGGL((truncate_kernel<false, false>), dim3(rows), dim3(kT), 0, st, ta);
  return launch_status("truncate_kernel");
}

int check_trunc_params(int64_t V, float temperature, int64_t top_k, float top_p) {
  TRIDA_CHECK(V > 0 && V < INT_MAX / 2, TRIDA_ERR_ARG, "V=%lld out of range", (long long)V);
  TRIDA_CHECK(temperature > 0.f && temperature < INFINITY, TRIDA_ERR_ARG,
              "temperature must be positive and finite (greedy decoding has its own entry point)");
  TRIDA_CHECK(top_p > 0.f && top_p <= 1.f, TRIDA_ERR_ARG, "top_p must lie in (0, 1]");
  TRIDA_CHECK(top_k >= 0, TRIDA_ERR_ARG, "top_k must be >= 0 (0 disables it)");
  TRIDA_CHECK(top_k == 0 || top_k >= V || top_k <= kMaxTopK, TRIDA_ERR_ARG, "top_k=%lld above the supported %d",
              (long long)top_k, kMaxTopK);
  return TRIDA_OK;
}

void plan_chunks(int64_t B, int64_t V, int* NC, int* chunk) {
  int64_t nc = std::min<int64_t>(64, std::max<int64_t>(1, cdiv(1024, B)));
  nc = std::min<int64_t>(nc, std::max<int64_t>(1, cdiv(V, 1024)));
  nc = std::max<int64_t>(nc, cdiv(V, kPickChunk));  // a chunk's weights fit the pick kernel's LDS
  *chunk = (int)cdiv(V, nc);
  *NC = (int)cdiv(V, *chunk);
}

struct ScratchLayout {
  int64_t m, thr, zk, status, state, rstatus, sums, total;
};
ScratchLayout layout(int64_t B, int64_t K, int64_t V) {
  int NC, chunk;
  plan_chunks(B, V, &NC, &chunk);
  const int64_t rows = B * (K + 1);
  ScratchLayout L;
  L.m = 0;
  L.thr = L.m + align_up(rows * 4, 256);
  L.zk = L.thr + align_up(rows * 4, 256);
  L.status = L.zk + align_up(rows * 8, 256);
  L.state = L.status + align_up(rows * 4, 256);
  L.rstatus = L.state + align_up(B * 4, 256);
  L.sums = L.rstatus + align_up(B * 4, 256);
  L.total = L.sums + align_up(B * NC * 2 * 8, 256);
  return L;
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_truncate_stats(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                                    int64_t row_stride, float temperature, int64_t top_k, float top_p,
                                    int64_t ban_id, int flags, float* m_out, float* thr_out, double* zk_out,
                                    int32_t* status_out, int32_t* passes_out, void* stream) {
  TRIDA_CHECK(logits && m_out && thr_out && zk_out && status_out, TRIDA_ERR_NULL, "null pointer argument");
  TRIDA_CHECK(B > 0 && R > 0 && B * R < INT_MAX, TRIDA_ERR_ARG, "bad B=%lld R=%lld", (long long)B, (long long)R);
  const int rc = check_trunc_params(V, temperature, top_k, top_p);
  if (rc != TRIDA_OK) return rc;
  TRIDA_CHECK(row_stride >= V && (B == 1 || batch_stride >= (R - 1) * row_stride + V), TRIDA_ERR_ARG,
              "strides too small");
  TruncArgs ta{logits, batch_stride, row_stride, (int)R, (int)V, 1.0 / (double)temperature, (int)top_k, top_p,
               ban_of(ban_id, V), flags, (int)R, 0, nullptr,
               m_out, thr_out, zk_out, status_out, passes_out};
  return launch_truncate(ta, (int)(B * R), vec_ok(logits, V, batch_stride, row_stride),
                         static_cast<hipStream_t>(stream));
}

extern "C" int64_t trida_sample_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int64_t K) {
  (void)R;
  if (B <= 0 || V <= 0 || K < 0) return -1;
  return layout(B, K, V).total;
}

extern "C" int trida_sample_accept(const float* p_logits, int64_t B, int64_t R, int64_t V, int64_t p_batch_stride,
                                   int64_t p_row_stride, const float* q_probs, int64_t q_batch_stride,
                                   int64_t q_row_stride, const int64_t* drafts, int64_t K, int64_t draft_stride,
                                   const int32_t* n_live, const float* u_accept, int64_t u_stride,
                                   const float* u_sample, const int64_t* ctx_len, float temperature, int64_t top_k,
                                   float top_p, int64_t ban_id, int32_t* n_acc, int64_t* token, int64_t* crop,
                                   double* ratio, int32_t* status, void* scratch, int64_t scratch_bytes,
                                   void* stream_) {
  hipStream_t stream = static_cast<hipStream_t>(stream_);
  TRIDA_CHECK(p_logits && u_sample && n_acc && token && crop && status && scratch, TRIDA_ERR_NULL,
              "null pointer argument");
  TRIDA_CHECK(K == 0 || (q_probs && drafts && u_accept), TRIDA_ERR_NULL, "q_probs, drafts and u_accept are needed when K > 0");
  TRIDA_CHECK(B > 0 && B <= 65535 && K >= 0 && K <= kWave && R >= K + 1, TRIDA_ERR_ARG,
              "need 0 < B <= 65535, 0 <= K <= 64 and R >= K + 1 (B=%lld K=%lld R=%lld)", (long long)B, (long long)K,
              (long long)R);
  const int rc = check_trunc_params(V, temperature, top_k, top_p);
  if (rc != TRIDA_OK) return rc;
  TRIDA_CHECK(p_row_stride >= V && (B == 1 || p_batch_stride >= (R - 1) * p_row_stride + V), TRIDA_ERR_ARG,
              "p strides too small");
  TRIDA_CHECK(K == 0 || (q_row_stride >= V && (B == 1 || (q_batch_stride >= (K - 1) * q_row_stride + V &&
                                                          draft_stride >= K && u_stride >= K))),
              TRIDA_ERR_ARG, "q / draft / uniform strides too small");
  const ScratchLayout L = layout(B, K, V);
  TRIDA_CHECK(scratch_bytes >= L.total, TRIDA_ERR_WORKSPACE, "scratch of %lld bytes, need %lld",
              (long long)scratch_bytes, (long long)L.total);
  TRIDA_CHECK((uintptr_t)scratch % 256 == 0, TRIDA_ERR_ALIGN, "scratch must be 256-byte aligned");
  char* s = static_cast<char*>(scratch);
  float* m = reinterpret_cast<float*>(s + L.m);
  float* thr = reinterpret_cast<float*>(s + L.thr);
  double* zk = reinterpret_cast<double*>(s + L.zk);
  int* st = reinterpret_cast<int*>(s + L.status);
  double* sums = reinterpret_cast<double*>(s + L.sums);

  int* state = reinterpret_cast<int*>(s + L.state);
  int* rstatus = reinterpret_cast<int*>(s + L.rstatus);
  int NC, chunk;
  plan_chunks(B, V, &NC, &chunk);
  AcceptArgs aa{p_logits, p_batch_stride, p_row_stride, q_probs, q_batch_stride, q_row_stride, drafts, draft_stride,
                n_live, u_accept, u_stride, u_sample, ctx_len, (int)B, (int)V, (int)K, 1.0 / (double)temperature,
                ban_of(ban_id, V), m, thr, zk, st, state, rstatus, NC, chunk, sums, n_acc, token, crop, ratio, status};

  // Only rows up to a sequence's first rejection decide anything. Rows 0..G0-1 of every sequence go
  // first (G0 sized so that this group alone fills the GPU, ~512 blocks); a one-wave scan per
  // sequence then settles the sequences it can, and one more group evaluates all the remaining rows
  // of the rest at once (decided sequences' blocks exit at once), followed by the final scan.
  const int R1 = (int)K + 1;
  const int G0 = (int)std::min<int64_t>(R1, std::max<int64_t>(8, cdiv(512, B)));
  const bool vec = vec_ok(p_logits, V, p_batch_stride, p_row_stride);
  int r = TRIDA_OK;
  for (int g = 0; g < 2; ++g) {
    const int first = g == 0 ? 0 : G0, cnt = g == 0 ? G0 : R1 - G0;
    if (cnt <= 0) break;
    TruncArgs ta{p_logits, p_batch_stride, p_row_stride, R1, (int)V, 1.0 / (double)temperature, (int)top_k, top_p,
                 ban_of(ban_id, V), 0, cnt, first, g > 0 ? state : nullptr, m, thr, zk, st, nullptr};
    r = launch_truncate(ta, (int)(B * cnt), vec, stream);
    if (r != TRIDA_OK) return r;
    hipLaunchKernelGGL(accept_scan_kernel, dim3(B), dim3(kWave), 0, stream, aa, first, cnt);
    r = launch_status("accept_scan_kernel");
    if (r != TRIDA_OK) return r;
  }
  hipLaunchKernelGGL(resid_sums_kernel, dim3(NC, B), dim3(kRT), 0, stream, aa);
  r = launch_status("resid_sums_kernel");
  if (r != TRIDA_OK) return r;
  hipLaunchKernelGGL(resid_pick_kernel, dim3(B), dim3(kRT), 0, stream, aa);
  return launch_status("resid_pick_kernel");
}

namespace trida {
namespace {
__global__ __launch_bounds__(256) void probs_kernel(const float* logits, int64_t bs, int64_t rs, int R, int V,
                                                    double rt, int ban, const float* m, const float* thr,
                                                    const double* zk, float* out, int64_t obs, int64_t ors) {
  const int r = blockIdx.y;
  const int b = r / R, i = r % R;
  const float* row = logits + (int64_t)b * bs + (int64_t)i * rs;
  float* o = out + (int64_t)b * obs + (int64_t)i * ors;
  const float mm = m[r], t = thr[r];
  const float inv = (float)(1.0 / zk[r]);
  for (int ix = blockIdx.x * 256 + threadIdx.x; ix < V; ix += gridDim.x * 256) {
    const float y = make_y<true>(row[ix], ix, rt, ban);
    o[ix] = (y > -INFINITY && y >= t) ? __expf(y - mm) * inv : 0.f;
  }
}
// Row-mapped form: out row out_rows[b K + j] of sequence b = P of logits row in_rows[b K + j] (whose
// statistics are at [b, in_rows[..]]). An index outside its range skips the row: the maps are device
// data the host cannot check. Four elements per thread per step (16-byte loads and stores) when vec.
template <bool kVec>
__global__ __launch_bounds__(256) void probs_rows_kernel(const float* logits, int64_t bs, int64_t rs, int R, int V,
                                                         double rt, int ban, const float* m, const float* thr,
                                                         const double* zk, const int64_t* in_rows,
                                                         const int64_t* out_rows, int K, int Ro, float* out,
                                                         int64_t obs, int64_t ors) {
  const int r = blockIdx.y;
  const int b = r / K;
  const int64_t i = in_rows[r], o = out_rows[r];
  if (i < 0 || i >= R || o < 0 || o >= Ro) return;  // block-uniform
  const float* row = logits + (int64_t)b * bs + i * rs;
  float* dst = out + (int64_t)b * obs + o * ors;
  const int64_t si = (int64_t)b * R + i;
  const float mm = m[si], t = thr[si];
  const float inv = (float)(1.0 / zk[si]);
  auto p_of = [&](float x, int ix) {
    const float y = make_y<true>(x, ix, rt, ban);
    return (y > -INFINITY && y >= t) ? __expf(y - mm) * inv : 0.f;
  };
  if (kVec) {
    const int n4 = V >> 2;
    for (int j = blockIdx.x * 256 + threadIdx.x; j < n4; j += gridDim.x * 256) {
      const u32x4 w = reinterpret_cast<const u32x4*>(row)[j];
      float4 y;
      y.x = p_of(__uint_as_float(w.x), 4 * j);
      y.y = p_of(__uint_as_float(w.y), 4 * j + 1);
      y.z = p_of(__uint_as_float(w.z), 4 * j + 2);
      y.w = p_of(__uint_as_float(w.w), 4 * j + 3);
      reinterpret_cast<float4*>(dst)[j] = y;
    }
  } else {
    for (int ix = blockIdx.x * 256 + threadIdx.x; ix < V; ix += gridDim.x * 256) dst[ix] = p_of(row[ix], ix);
  }
}

// dst[b, k, :] = fp32(src[b, rows[b, k], :]) for bf16 (kBf16) or fp32 sources; a row index outside
// [0, R) skips the row. 16-byte loads and stores when vec (8 bf16 or 4 fp32 elements a load).
template <bool kBf16, bool kVec>
__global__ __launch_bounds__(256) void gather_rows_kernel(const void* src, int64_t sbs, int64_t srs, int R, int V,
                                                          const int64_t* rows, int K, float* dst, int64_t dbs,
                                                          int64_t drs) {
  const int r = blockIdx.y;
  const int b = r / K, k = r % K;
  const int64_t i = rows[r];
  if (i < 0 || i >= R) return;  // block-uniform
  float* d = dst + (int64_t)b * dbs + (int64_t)k * drs;
  const int64_t off = (int64_t)b * sbs + i * srs;
  if (kBf16) {
    const uint16_t* s = static_cast<const uint16_t*>(src) + off;
    if (kVec) {
      for (int j = blockIdx.x * 256 + threadIdx.x; j < (V >> 3); j += gridDim.x * 256) {
        const u32x4 w = reinterpret_cast<const u32x4*>(s)[j];
        float4 lo, hi;
        lo.x = __uint_as_float(w.x << 16);
        lo.y = __uint_as_float(w.x & 0xffff0000u);
        lo.z = __uint_as_float(w.y << 16);
        lo.w = __uint_as_float(w.y & 0xffff0000u);
        hi.x = __uint_as_float(w.z << 16);
        hi.y = __uint_as_float(w.z & 0xffff0000u);
        hi.z = __uint_as_float(w.w << 16);
        hi.w = __uint_as_float(w.w & 0xffff0000u);
        reinterpret_cast<float4*>(d)[2 * j] = lo;
        reinterpret_cast<float4*>(d)[2 * j + 1] = hi;
      }
    } else {
      for (int ix = blockIdx.x * 256 + threadIdx.x; ix < V; ix += gridDim.x * 256) d[ix] = bf2f(s[ix]);
    }
  } else {
    const float* s = static_cast<const float*>(src) + off;
    if (kVec) {
      for (int j = blockIdx.x * 256 + threadIdx.x; j < (V >> 2); j += gridDim.x * 256)
        reinterpret_cast<float4*>(d)[j] = reinterpret_cast<const float4*>(s)[j];
    } else {
      for (int ix = blockIdx.x * 256 + threadIdx.x; ix < V; ix += gridDim.x * 256) d[ix] = s[ix];
    }
  }
}
}  // namespace
}  // namespace trida

extern "C" int trida_truncated_probs_rows(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                                          int64_t row_stride, float temperature, int64_t ban_id, const float* m,
                                          const float* thr, const double* zk, const int64_t* in_rows,
                                          const int64_t* out_rows, int64_t K, float* probs, int64_t Ro,
                                          int64_t out_batch_stride, int64_t out_row_stride, void* stream) {
  TRIDA_CHECK(logits && m && thr && zk && in_rows && out_rows && probs, TRIDA_ERR_NULL, "null pointer argument");
  TRIDA_CHECK(B > 0 && R > 0 && K >= 0 && Ro > 0 && B * K <= 65535 && V > 0 && V < INT_MAX / 2, TRIDA_ERR_ARG,
              "bad shape");
  TRIDA_CHECK(temperature > 0.f && temperature < INFINITY, TRIDA_ERR_ARG, "temperature must be positive");
  TRIDA_CHECK(row_stride >= V && out_row_stride >= V &&
                  (B == 1 || (batch_stride >= (R - 1) * row_stride + V &&
                              out_batch_stride >= (Ro - 1) * out_row_stride + V)),
              TRIDA_ERR_ARG, "strides too small");
  if (K == 0) return TRIDA_OK;
  const bool vec = V % 4 == 0 && row_stride % 4 == 0 && batch_stride % 4 == 0 && out_row_stride % 4 == 0 &&
                   out_batch_stride % 4 == 0 && (((uintptr_t)logits | (uintptr_t)probs) & 15) == 0;
  const int gx = (int)std::min<int64_t>(cdiv(V, 256 * (vec ? 4 : 1)), 256);
  const dim3 grid(gx, (unsigned)(B * K));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL((probs_rows_kernel<true>), grid, dim3(256), 0, st, logits, batch_stride, row_stride, (int)R,
                       (int)V, 1.0 / (double)temperature, ban_of(ban_id, V), m, thr, zk, in_rows, out_rows, (int)K,
                       (int)Ro, probs, out_batch_stride, out_row_stride);
  else
    hipLaunchKernelGGL((probs_rows_kernel<false>), grid, dim3(256), 0, st, logits, batch_stride, row_stride, (int)R,
                       (int)V, 1.0 / (double)temperature, ban_of(ban_id, V), m, thr, zk, in_rows, out_rows, (int)K,
                       (int)Ro, probs, out_batch_stride, out_row_stride);
  return launch_status("probs_rows_kernel");
}

extern "C" int trida_gather_rows(const void* src, int dtype, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                                 int64_t row_stride, const int64_t* rows, int64_t K, float* dst,
                                 int64_t out_batch_stride, int64_t out_row_stride, void* stream) {
  TRIDA_CHECK(src && rows && dst, TRIDA_ERR_NULL, "null pointer argument");
  TRIDA_CHECK(dtype == 0 || dtype == 1, TRIDA_ERR_ARG, "dtype must be 0 (fp32) or 1 (bf16)");
  TRIDA_CHECK(B > 0 && R > 0 && K >= 0 && B * K <= 65535 && V > 0 && V < INT_MAX / 2, TRIDA_ERR_ARG, "bad shape");
  TRIDA_CHECK(row_stride >= V && out_row_stride >= V &&
                  (B == 1 || (batch_stride >= (R - 1) * row_stride + V &&
                              out_batch_stride >= (K - 1) * out_row_stride + V)),
              TRIDA_ERR_ARG, "strides too small");
  if (K == 0) return TRIDA_OK;
  const int e = dtype == 1 ? 8 : 4;  // elements per 16-byte load
  const bool vec = V % e == 0 && row_stride % e == 0 && batch_stride % e == 0 && out_row_stride % 4 == 0 &&
                   out_batch_stride % 4 == 0 && (((uintptr_t)src | (uintptr_t)dst) & 15) == 0;
  const int gx = (int)std::min<int64_t>(cdiv(V, 256 * (vec ? e : 1)), 256);
  const dim3 grid(gx, (unsigned)(B * K));
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == 1 && vec)
    hipLaunchKernelGGL((gather_rows_kernel<true, true>), grid, dim3(256), 0, st, src, batch_stride, row_stride, (int)R,
                       (int)V, rows, (int)K, dst, out_batch_stride, out_row_stride);
  else if (dtype == 1)
    hipLaunchKernelGGL((gather_rows_kernel<true, false>), grid, dim3(256), 0, st, src, batch_stride, row_stride,
                       (int)R, (int)V, rows, (int)K, dst, out_batch_stride, out_row_stride);
  else if (vec)
    hipLaunchKernelGGL((gather_rows_kernel<false, true>), grid, dim3(256), 0, st, src, batch_stride, row_stride,
                       (int)R, (int)V, rows, (int)K, dst, out_batch_stride, out_row_stride);
  else
    hipLaunchKernelGGL((gather_rows_kernel<false, false>), grid, dim3(256), 0, st, src, batch_stride, row_stride,
                       (int)R, (int)V, rows, (int)K, dst, out_batch_stride, out_row_stride);
  return launch_status("gather_rows_kernel");
}

extern "C" int trida_truncated_probs(const float* logits, int64_t B, int64_t R, int64_t V, int64_t batch_stride,
                                     int64_t row_stride, float temperature, int64_t ban_id, const float* m,
                                     const float* thr, const double* zk, float* probs, int64_t out_batch_stride,
                                     int64_t out_row_stride, void* stream) {
  TRIDA_CHECK(logits && m && thr && zk && probs, TRIDA_ERR_NULL, "null pointer argument");
  TRIDA_CHECK(B > 0 && R > 0 && B * R <= 65535 && V > 0 && V < INT_MAX / 2, TRIDA_ERR_ARG, "bad shape");
  TRIDA_CHECK(temperature > 0.f && temperature < INFINITY, TRIDA_ERR_ARG, "temperature must be positive");
  TRIDA_CHECK(row_stride >= V && out_row_stride >= V &&
                  (B == 1 || (batch_stride >= (R - 1) * row_stride + V &&
                              out_batch_stride >= (R - 1) * out_row_stride + V)),
              TRIDA_ERR_ARG, "strides too small");
  const int gx = (int)std::min<int64_t>(cdiv(V, 256 * 8), 256);
  hipLaunchKernelGGL(probs_kernel, dim3(gx, B * R), dim3(256), 0, static_cast<hipStream_t>(stream), logits, batch_stride, row_stride, (int)R,
                     (int)V, 1.0 / (double)temperature, ban_of(ban_id, V), m, thr, zk, probs, out_batch_stride, out_row_stride);
  return launch_status("probs_kernel");
}

// ---------------------------------------------------------------- draws from given truncation statistics
// The residual kernels with no drafts: per row, the inverse CDF in vocabulary order of
// P(x) = [y_x >= thr] exp(y_x - m) / zk at one uniform. Scratch: the per-row bookkeeping those kernels
// read and write, then the chunk sums.
namespace trida {
namespace {
struct DrawScratch {
  int64_t state, rstatus, status, n_acc, crop, sums, total;
};
DrawScratch draw_layout(int64_t rows, int64_t V) {
  int NC, chunk;
  plan_chunks(rows, V, &NC, &chunk);
  DrawScratch L;
  L.state = 0;
  L.rstatus = L.state + align_up(rows * 4, 256);
  L.status = L.rstatus + align_up(rows * 4, 256);
  L.n_acc = L.status + align_up(rows * 4, 256);
  L.crop = L.n_acc + align_up(rows * 4, 256);
  L.sums = L.crop + align_up(rows * 8, 256);
  L.total = L.sums + align_up(rows * NC * 2 * 8, 256);
  return L;
}
}  // namespace
}  // namespace trida

extern "C" int64_t trida_sample_rows_scratch_bytes(int64_t rows, int64_t V) {
  if (rows <= 0 || V <= 0) return 0;
  return draw_layout(rows, V).total;
}

extern "C" int trida_sample_rows(const float* logits, int64_t rows, int64_t V, int64_t row_stride, float temperature,
                                 int64_t ban_id, const float* m, const float* thr, const double* zk, const float* u,
                                 int64_t* token, void* scratch, int64_t scratch_bytes, void* stream) {
  TRIDA_CHECK(logits && m && thr && zk && u && token && scratch, TRIDA_ERR_NULL, "null pointer argument");
  TRIDA_CHECK(rows > 0 && rows <= 65535 && V > 0 && V < INT_MAX / 2, TRIDA_ERR_ARG, "bad shape rows=%lld V=%lld",
              (long long)rows, (long long)V);
  TRIDA_CHECK(temperature > 0.f && temperature < INFINITY, TRIDA_ERR_ARG, "temperature must be positive");
  TRIDA_CHECK(row_stride >= V, TRIDA_ERR_ARG, "row_stride too small");
  const DrawScratch L = draw_layout(rows, V);
  TRIDA_CHECK(scratch_bytes >= L.total, TRIDA_ERR_WORKSPACE, "scratch of %lld bytes, need %lld",
              (long long)scratch_bytes, (long long)L.total);
  TRIDA_CHECK((uintptr_t)scratch % 256 == 0, TRIDA_ERR_ALIGN, "scratch must be 256-byte aligned");
  char* s = static_cast<char*>(scratch);
  int NC, chunk;
  plan_chunks(rows, V, &NC, &chunk);
  AcceptArgs aa{logits, row_stride, 0, nullptr, 0, 0, nullptr, 0, nullptr, nullptr, 0, u, nullptr, (int)rows, (int)V, 0,
                1.0 / (double)temperature, ban_of(ban_id, V), m, thr, zk, nullptr,
                reinterpret_cast<int*>(s + L.state), reinterpret_cast<int*>(s + L.rstatus), NC, chunk,
                reinterpret_cast<double*>(s + L.sums), reinterpret_cast<int32_t*>(s + L.n_acc), token,
                reinterpret_cast<int64_t*>(s + L.crop), nullptr, reinterpret_cast<int32_t*>(s + L.status)};
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(resid_sums_kernel, dim3(NC, rows), dim3(kRT), 0, st, aa);
  const int r = launch_status("resid_sums_kernel (draw)");
  if (r != TRIDA_OK) return r;
  hipLaunchKernelGGL(resid_pick_kernel, dim3(rows), dim3(kRT), 0, st, aa);
  return launch_status("resid_pick_kernel (draw)");
}
