// Greedy self-spec acceptance: one HBM pass over the verify logits, then a per-sequence prefix scan.
//
// Two launches on the caller's stream, no atomics:
//   split_argmax (grid S x R x B): block (s, r, b) reduces split s of row r of sequence b to an
//       (argmax value, index) pair in scratch. Each thread issues U 16-byte nontemporal loads per tile
//       back to back (indices clamped in bounds, compares masked), so a block has U * 4 KiB in flight.
//   finalize (grid B): stages the split results and the drafts through LDS (one memory latency per
//       pass), reduces each row with one thread per row, then one wave ballots draft matches and
//       takes the accepted length as the count of leading ones.
// A single-launch variant that elected the last block with device-scope counters measured slower on
// gfx950: every arrive costs a device-scope atomic round trip (~20 ns each, serialised), which for
// ~600 blocks exceeds the whole streaming pass.
#include <limits.h>
#include <math.h>

#include "common.h"

namespace trida {
namespace {

constexpr int kThreads = 256;
constexpr int kStage = 2048;  // split results staged per pass by finalize (a pass holds whole rows)

// (a, ia) ranks above (b, ib): NaN above everything, then larger value, then smaller index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na | nb) return na && (!nb || ia < ib);
  return (a > b) || (a == b && ia < ib);
}

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
  const float* logits;
  int64_t batch_stride, row_stride;
  int V, R, S, chunk;
  float* pval;
  int* pidx;
};

template <int U, bool kVec>
__global__ __launch_bounds__(kThreads) void split_argmax_kernel(SplitArgs a) {
  const int s = blockIdx.x, r = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const float* row = a.logits + (int64_t)b * a.batch_stride + (int64_t)r * a.row_stride;
  const int lo = s * a.chunk;
  const int hi = min(a.V, lo + a.chunk);

  float best = -INFINITY;
  int bi = INT_MAX;
  if (kVec) {
    // lo is a multiple of 4 and the row start is 16-byte aligned (checked on the host)
    const f32x4* row4 = reinterpret_cast<const f32x4*>(row + lo);
    const int n4 = (hi - lo) >> 2;
    for (int base = 0; base < n4; base += kThreads * U) {
      f32x4 x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = __builtin_nontemporal_load(row4 + min(base + u * kThreads + tid, n4 - 1));
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = base + u * kThreads + tid;
        const bool ok = j < n4;
        const int ix = lo + 4 * j;
        take(x[u].x, ix, ok, best, bi);
        take(x[u].y, ix + 1, ok, best, bi);
        take(x[u].z, ix + 2, ok, best, bi);
        take(x[u].w, ix + 3, ok, best, bi);
      }
    }
    for (int ix = lo + 4 * n4 + tid; ix < hi; ix += kThreads) take(row[ix], ix, true, best, bi);
  } else {
    for (int ix = lo + tid; ix < hi; ix += kThreads) take(row[ix], ix, true, best, bi);
  }

  __shared__ float sv[kThreads / kWave];
  __shared__ int si[kThreads / kWave];
  wave_argbest(best, bi);
  const int wave = tid / kWave, lane = tid % kWave;
  if (lane == 0) {
    sv[wave] = best;
    si[wave] = bi;
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

  // wave 0: prefix scan of draft matches (ballot; accepted = count of leading ones)
  if (wave == 0) {
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

// Split a row into chunks of one tile each (kThreads * U float4), U in {4, 8, 16}: the largest U
// that still gives at least ~512 blocks; callers may force the split count.
void plan(int64_t B, int64_t R, int64_t V, int64_t splits_req, int64_t* S, int64_t* chunk) {
  int64_t c;
  if (splits_req > 0) {
    c = align_up(cdiv(V, splits_req), 4);
  } else {
    c = 4 * kThreads * 4;
    for (int u = 16; u >= 4; u /= 2) {
      c = 4 * kThreads * u;
      if (B * R * cdiv(V, c) >= 512) break;
    }
  }
  *chunk = c;
  *S = cdiv(V, c);
}

int pick_unroll(int64_t chunk) {
  const int64_t per_thread = cdiv(chunk / 4, kThreads);
  return per_thread <= 4 ? 4 : (per_thread <= 8 ? 8 : 16);
}

int64_t scratch_bytes(int64_t B, int64_t R, int64_t S) { return align_up(B * R * S * 4, 256) * 2; }

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_greedy_accept_scratch_bytes(int64_t B, int64_t R, int64_t V, int64_t splits) {
  if (B <= 0 || R <= 0 || V <= 0) return 0;
  int64_t S, chunk;
  plan(B, R, V, splits, &S, &chunk);
  return scratch_bytes(B, R, S);
}

extern "C" int trida_greedy_accept(const float* logits, int64_t B, int64_t R, int64_t V,
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
  int64_t S, chunk;
  plan(B, R, V, splits, &S, &chunk);
  TRIDA_CHECK(S <= kStage && S <= 65535, TRIDA_ERR_ARG, "greedy_accept: at most %d splits per row", kStage);
  TRIDA_CHECK(scratch_bytes_ >= scratch_bytes(B, R, S), TRIDA_ERR_WORKSPACE,
              "greedy_accept: scratch %lld < %lld bytes", (long long)scratch_bytes_,
              (long long)scratch_bytes(B, R, S));
  char* ws = static_cast<char*>(scratch);
  float* pval = reinterpret_cast<float*>(ws);
  int* pidx = reinterpret_cast<int*>(ws + align_up(B * R * S * 4, 256));
  hipStream_t st = static_cast<hipStream_t>(stream);

  SplitArgs sa{logits, batch_stride, row_stride, (int)V, (int)R, (int)S, (int)chunk, pval, pidx};
  const bool vec = ((reinterpret_cast<uintptr_t>(logits) & 15) == 0) && (row_stride % 4 == 0) &&
                   (batch_stride % 4 == 0);
  dim3 grid((unsigned)S, (unsigned)R, (unsigned)B);
  if (!vec) {
    hipLaunchKernelGGL((split_argmax_kernel<4, false>), grid, dim3(kThreads), 0, st, sa);
  } else {
    switch (pick_unroll(chunk)) {
      case 4: hipLaunchKernelGGL((split_argmax_kernel<4, true>), grid, dim3(kThreads), 0, st, sa); break;
      case 8: hipLaunchKernelGGL((split_argmax_kernel<8, true>), grid, dim3(kThreads), 0, st, sa); break;
      default: hipLaunchKernelGGL((split_argmax_kernel<16, true>), grid, dim3(kThreads), 0, st, sa); break;
    }
  }
  int rc = launch_status("greedy_accept/split_argmax");
  if (rc) return rc;
  FinalArgs fa{pval, pidx, (int)R, (int)S, drafts, draft_stride, (int)K, n_live, ctx_len,
               argmax_out, n_acc, bonus, crop};
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)B), dim3(kThreads), 0, st, fa);
  return launch_status("greedy_accept/finalize");
}
