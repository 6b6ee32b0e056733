// Banned and gated tokens, applied in place to logit rows before an argmax or a sampling kernel reads
// them: the two steps of apply_ban (inference/zoro-1/mlx/trida_mlx/decode.py:76-99).
//   ban:  x[r, id] = -inf for every listed id (the bias of -inf the reference adds).
//   gate: per row, lse = logsumexp(x[r, :]) over the (banned) row; for each gate (id, thr),
//         p = exp(x[r, id] - lse), and x[r, id] = -inf where p < thr. Every p of a row is taken before
//         any gate of that row writes (the reference computes lse once, before its gate loop).
// The gate reads each row once: one workgroup per row keeps an online (max, sum of exp) per thread,
// merged across the workgroup, then thread g handles gate g.
#include <math.h>

#include "common.h"

namespace trida {
namespace {

constexpr int kBanThreads = 256;
constexpr int kGateThreads = 512;

template <typename T>
__device__ __forceinline__ float load_x(const T* p);
template <>
__device__ __forceinline__ float load_x<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_x<uint16_t>(const uint16_t* p) { return bf2f(*p); }

template <typename T>
__device__ __forceinline__ void store_ninf(T* p);
template <>
__device__ __forceinline__ void store_ninf<float>(float* p) { *p = -INFINITY; }
template <>
__device__ __forceinline__ void store_ninf<uint16_t>(uint16_t* p) { *p = 0xff80u; }

template <typename T>
__global__ __launch_bounds__(kBanThreads) void ban_kernel(T* x, int64_t row_stride, int V, const int64_t* ids,
                                                          int n_ids) {
  const int j = blockIdx.x * kBanThreads + threadIdx.x;
  if (j >= n_ids) return;
  const int64_t id = ids[j];
  if (id < 0 || id >= V) return;
  store_ninf(x + (int64_t)blockIdx.y * row_stride + id);
}

// Online (m, s) pair: s = sum exp(v - m) over the values seen; -inf values add nothing.
__device__ __forceinline__ void lse_add(float v, float& m, float& s) {
  if (v == -INFINITY || v != v) {
    if (v != v) m = v;  // a NaN row stays NaN
    return;
  }
  if (v > m) {
    s = s * __expf(m - v) + 1.f;
    m = v;
  } else {
    s += (v == m) ? 1.f : __expf(v - m);  // equal infinities add exp(0)
  }
}

__device__ __forceinline__ void lse_merge(float& m, float& s, float om, float os) {
  if (m != m || om != om) {
    m = NAN;
    return;
  }
  const float nm = fmaxf(m, om);
  if (nm == -INFINITY) return;
  s = s * (m == nm ? 1.f : __expf(m - nm)) + os * (om == nm ? 1.f : __expf(om - nm));
  m = nm;
}

template <typename T>
__global__ __launch_bounds__(kGateThreads) void gate_kernel(T* x, int64_t row_stride, int V, const int64_t* ids,
                                                            const float* thr, int n_gate, float* raw_p) {
  T* row = x + (int64_t)blockIdx.x * row_stride;
  float m = -INFINITY, s = 0.f;
  for (int i = threadIdx.x; i < V; i += kGateThreads) lse_add(load_x(row + i), m, s);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off, kWave), os = __shfl_xor(s, off, kWave);
    lse_merge(m, s, om, os);
  }
  __shared__ float sm[kGateThreads / kWave], ss[kGateThreads / kWave];
  __shared__ float s_lse;
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) {
    sm[wave] = m;
    ss[wave] = s;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float M = sm[0], S = ss[0];
    for (int w = 1; w < kGateThreads / kWave; ++w) lse_merge(M, S, sm[w], ss[w]);
    s_lse = (M == -INFINITY) ? -INFINITY : M + __logf(S);
  }
  __syncthreads();
  const float lse = s_lse;
  // every p of the row before any write (gates on the same id see the unwritten value)
  float p = 0.f;
  int64_t id = -1;
  if ((int)threadIdx.x < n_gate) {
    id = ids[threadIdx.x];
    if (id >= 0 && id < V && lse != -INFINITY) p = __expf(load_x(row + id) - lse);
    if (raw_p) raw_p[(int64_t)blockIdx.x * n_gate + threadIdx.x] = p;
  }
  if (!thr) return;  // a note-only pass: the raw probabilities, nothing written to the row
  __syncthreads();
  if ((int)threadIdx.x < n_gate && id >= 0 && id < V && thr[threadIdx.x] > 0.f && p < thr[threadIdx.x])
    store_ninf(row + id);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_ban_tokens(void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                                const int64_t* ids, int64_t n_ids, void* stream) {
  TRIDA_CHECK(dtype == 0 || dtype == 1, TRIDA_ERR_ARG, "ban_tokens: logits dtype must be 0 (fp32) or 1 (bf16)");
  TRIDA_CHECK(rows >= 0 && rows <= 65535 && V > 0 && V < INT32_MAX && row_stride >= V && n_ids >= 0 &&
                  n_ids < INT32_MAX,
              TRIDA_ERR_ARG, "ban_tokens: bad sizes rows=%lld V=%lld n_ids=%lld", (long long)rows, (long long)V,
              (long long)n_ids);
  if (rows == 0 || n_ids == 0) return TRIDA_OK;
  TRIDA_CHECK(logits && ids, TRIDA_ERR_NULL, "ban_tokens: logits and ids are required");
  const dim3 grid((unsigned)cdiv(n_ids, kBanThreads), (unsigned)rows);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    hipLaunchKernelGGL(ban_kernel<float>, grid, dim3(kBanThreads), 0, st, static_cast<float*>(logits), row_stride,
                       (int)V, ids, (int)n_ids);
  else
    hipLaunchKernelGGL(ban_kernel<uint16_t>, grid, dim3(kBanThreads), 0, st, static_cast<uint16_t*>(logits),
                       row_stride, (int)V, ids, (int)n_ids);
  return launch_status("ban_tokens");
}

extern "C" int trida_gate_tokens(void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                                 const int64_t* ids, const float* thr, int64_t n_gate, float* raw_p, void* stream) {
  TRIDA_CHECK(dtype == 0 || dtype == 1, TRIDA_ERR_ARG, "gate_tokens: logits dtype must be 0 (fp32) or 1 (bf16)");
  TRIDA_CHECK(rows >= 0 && rows < INT32_MAX && V > 0 && V < INT32_MAX && row_stride >= V && n_gate >= 0 &&
                  n_gate <= kGateThreads,
              TRIDA_ERR_ARG, "gate_tokens: bad sizes rows=%lld V=%lld n_gate=%lld (<= %d)", (long long)rows,
              (long long)V, (long long)n_gate, kGateThreads);
  if (rows == 0 || n_gate == 0) return TRIDA_OK;
  TRIDA_CHECK(logits && ids && (thr || raw_p), TRIDA_ERR_NULL,
              "gate_tokens: logits, ids and thr (or, for a note-only pass, raw_p) are required");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (dtype == 0)
    hipLaunchKernelGGL(gate_kernel<float>, dim3((unsigned)rows), dim3(kGateThreads), 0, st,
                       static_cast<float*>(logits), row_stride, (int)V, ids, thr, (int)n_gate, raw_p);
  else
    hipLaunchKernelGGL(gate_kernel<uint16_t>, dim3((unsigned)rows), dim3(kGateThreads), 0, st,
                       static_cast<uint16_t*>(logits), row_stride, (int)V, ids, thr, (int)n_gate, raw_p);
  return launch_status("gate_tokens");
}
