// Shared device helpers and host-side error plumbing for the gfx950 kernels behind include/trida_hip.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/trida_hip.h"

namespace trida {

// ---------------------------------------------------------------- bf16 storage (uint16 bits)
// Round-to-nearest-even, quiet NaN preserved: the same rounding torch applies on fp32 -> bf16. gfx950's
// v_cvt_pk_bf16_f32 does it in one instruction (two values for f2bf2); checked on every one of the 2^32
// fp32 inputs against (u + 0x7fff + ((u >> 16) & 1)) >> 16, with NaNs quieted as (u >> 16) | 0x40.
typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {  // lo in bits 0..15, hi in 16..31
  const f32x2v v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v));
}
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- wave64 helpers
constexpr int kWave = 64;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}
// Sum across aligned groups of `width` lanes (width a power of two <= 64).
template <int width>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = width / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// Device-scope release/acquire used by the last-block-done reductions. On gfx950 these lower to the
// L2 write-back / invalidate that make one XCD's stores visible to a block running on another XCD.
// Arrive with release only: the acquire (an L2 invalidate on gfx950) is paid once, by the block
// that finds itself last, through fence_acquire().
__device__ __forceinline__ unsigned arrive_release(unsigned* counter) {
  return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void fence_acquire() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }
__device__ __forceinline__ void reset_counter(unsigned* counter) {
  __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroups are dispatched to the 8 XCDs round-robin (block i runs on XCD i % 8), each XCD with its
// own L2. xcd_major(i, n) renumbers the n blocks of a grid so that logical ids [x n/8, (x + 1) n/8)
// all run on XCD x: neighbouring logical units, which read the same operands, then share one L2.
// A bijection on [0, n); the identity unless n is a multiple of 8.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_major(int i, int n) {
  return (n % kXcds) ? i : (i % kXcds) * (n / kXcds) + i / kXcds;
}

// Fragment order of the weight-streaming GEMM's activations X [M <= 48, K]: per k-step s of 32 columns and
// m-tile mt of 16 rows, 64 lanes x 16 bytes, lane 16 g + r holding X[16 mt + r][32 s + 8 g .. + 8] (the
// B operand of v_mfma_f32_16x16x32_bf16 as it lands in a register). Element offset of X[m][k]:
constexpr int kWsFragMT = 3;  // m-tiles per k-step, whatever M is
__host__ __device__ inline int64_t ws_frag_off(int m, int64_t k) {
  return (((k / 32) * kWsFragMT + m / 16) * 64 + ((k % 32) / 8) * 16 + m % 16) * 8 + k % 8;
}

// Argmax order of (value, index) pairs: NaN above every number (the first NaN wins), then the larger
// value, then the smaller index -- torch.argmax's first-index result, NaN included.
__device__ __forceinline__ bool argmax_better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na | nb) return na && (!nb || ia < ib);
  return (a > b) || (a == b && ia < ib);
}

// Online softmax denominator over the elements one thread has seen: s = sum exp(x - m) (NaN skipped).
__device__ __forceinline__ void acc_exp(float x, bool valid, float& m, float& s) {
  if (!valid || x != x) return;
  if (x > m) {
    s = s * __expf(m - x) + 1.f;
    m = x;
  } else {
    s += __expf(x - m);
  }
}
// Two such (m, s) states merged into (m, s).
__device__ __forceinline__ void merge_exp(float& m, float& s, float om, float os) {
  const float nm = fmaxf(m, om);
  s = (nm == -INFINITY) ? 0.f : s * __expf(m - nm) + os * __expf(om - nm);
  m = nm;
}

// ---------------------------------------------------------------- host error plumbing
void set_error(const char* fmt, ...);
int launch_status(const char* what);

inline int64_t align_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace trida

#define TRIDA_CHECK(cond, code, ...)      \
  do {                                    \
    if (!(cond)) {                        \
      trida::set_error(__VA_ARGS__);      \
      return (code);                      \
    }                                     \
  } while (0)
