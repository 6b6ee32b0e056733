// Skinny bf16 GEMM for the decode-step projections: Y[M, N] = X[M, K] W[N, K]^T with M <= 64
// (a canvas of <= 64 rows), fp32 accumulation, bf16 output. At these M the GEMM is bound by the weight
// stream, so the kernel is built to read every weight byte exactly once at full HBM rate:
//   - a wave owns 16 weight rows (the MFMA A operand, 16-byte nontemporal loads, 8 k-steps in flight)
//     and every activation row (B operand, MT tiles of 16 rows; X is small and stays in L2);
//   - v_mfma_f32_16x16x32_bf16 accumulates C^T[n, m];
//   - the 4 waves of a workgroup split K and reduce through LDS; when N is small the grid also splits
//     K across workgroups (fp32 partials, then a reduce kernel), so the launch covers all CUs.
#include "common.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ bf16x8 as_bf(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

constexpr int kNW = 4;
constexpr int kU = 8;  // k-steps (32 k each) in flight per wave

struct GemmArgs {
  const uint16_t* X;
  const uint16_t* W;
  uint16_t* Y;
  float* partial;  // [SK, M, N] when SK > 1
  int64_t x_st, w_st, y_st;
  int M, N, K, SK;
};

template <int MT>
__global__ __launch_bounds__(kNW* kWave) void skinny_gemm_kernel(GemmArgs a) {
  const int nt = blockIdx.x, sk = blockIdx.y;
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int ksteps = a.K / 32;
  const int part = sk * kNW + wave, nparts = a.SK * kNW;
  const int s0 = (int)((int64_t)ksteps * part / nparts);
  const int s1 = (int)((int64_t)ksteps * (part + 1) / nparts);
  const int n = nt * 16 + (l % 16);
  const u32x4* wrow = reinterpret_cast<const u32x4*>(a.W + (int64_t)n * a.w_st + (l / 16) * 8);
  const u32x4* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + (l % 16), a.M - 1);  // rows past M repeat the last row; never stored
    xrow[mt] = reinterpret_cast<const u32x4*>(a.X + (int64_t)m * a.x_st + (l / 16) * 8);
  }
  f32x4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int s = s0;
  for (; s + kU <= s1; s += kU) {
    u32x4 wv[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) wv[u] = __builtin_nontemporal_load(wrow + (int64_t)(s + u) * 4);
    u32x4 xv[kU][MT];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[u][mt] = xrow[mt][(int64_t)(s + u) * 4];
#pragma unroll
    for (int u = 0; u < kU; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(wv[u]), as_bf(xv[u][mt]), acc[mt], 0, 0, 0);
  }
  for (; s < s1; ++s) {
    const u32x4 wv = __builtin_nontemporal_load(wrow + (int64_t)s * 4);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
      acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(wv), as_bf(xrow[mt][(int64_t)s * 4]), acc[mt], 0, 0, 0);
  }

  // reduce the 4 waves' K quarters; lane l holds C^T[n = (l/16)*4 + i][m = mt*16 + l%16]
  __shared__ f32x4 red[kNW - 1][MT][kWave];
  if (wave > 0)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave - 1][mt][l] = acc[mt];
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < kNW - 1; ++w)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] += red[w][mt][l];
  const int n0 = nt * 16 + (l / 16) * 4;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + (l % 16);
    if (m >= a.M) continue;
    if (a.SK == 1) {
      u32x2 packed;
      packed.x = (uint32_t)f2bf(acc[mt].x) | ((uint32_t)f2bf(acc[mt].y) << 16);
      packed.y = (uint32_t)f2bf(acc[mt].z) | ((uint32_t)f2bf(acc[mt].w) << 16);
      *reinterpret_cast<u32x2*>(a.Y + (int64_t)m * a.y_st + n0) = packed;
    } else {
      *reinterpret_cast<f32x4*>(a.partial + ((int64_t)sk * a.M + m) * a.N + n0) = acc[mt];
    }
  }
}

__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* partial, uint16_t* Y, int64_t y_st, int M, int N,
                                                            int SK) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one thread per 4 outputs
  if (i >= (int64_t)M * N / 4) return;
  const int m = (int)(i / (N / 4)), n = (int)(i % (N / 4)) * 4;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < SK; ++k) s += *reinterpret_cast<const f32x4*>(partial + ((int64_t)k * M + m) * N + n);
  u32x2 packed;
  packed.x = (uint32_t)f2bf(s.x) | ((uint32_t)f2bf(s.y) << 16);
  packed.y = (uint32_t)f2bf(s.z) | ((uint32_t)f2bf(s.w) << 16);
  *reinterpret_cast<u32x2*>(Y + (int64_t)m * y_st + n) = packed;
}

int plan_sk(int64_t N, int64_t K, int64_t splits) {
  if (splits > 0) return (int)splits;
  const int64_t tiles = N / 16, ksteps = K / 32;
  int64_t sk = cdiv(1024, tiles);
  const int64_t cap = ksteps / (kNW * 2);  // at least ~2 k-steps per wave
  if (sk > cap) sk = cap;
  return (int)(sk < 1 ? 1 : sk);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_skinny_gemm_scratch_bytes(int64_t M, int64_t N, int64_t K, int64_t splits) {
  const int sk = plan_sk(N, K, splits);
  return sk > 1 ? align_up((int64_t)sk * M * N * 4, 256) : 0;
}

extern "C" int trida_skinny_gemm(const uint16_t* X, int64_t x_row_stride, const uint16_t* W, int64_t w_row_stride,
                                 uint16_t* Y, int64_t y_row_stride, int64_t M, int64_t N, int64_t K, void* scratch,
                                 int64_t scratch_bytes, int64_t splits, void* stream) {
  TRIDA_CHECK(X && W && Y, TRIDA_ERR_NULL, "skinny_gemm: X, W and Y are required");
  TRIDA_CHECK(M >= 1 && M <= 64 && N > 0 && N % 16 == 0 && K > 0 && K % 32 == 0, TRIDA_ERR_ARG,
              "skinny_gemm: need 1 <= M <= 64, N % 16 == 0, K % 32 == 0 (M=%lld N=%lld K=%lld)", (long long)M,
              (long long)N, (long long)K);
  TRIDA_CHECK(x_row_stride >= K && w_row_stride >= K && y_row_stride >= N && x_row_stride % 8 == 0 &&
                  w_row_stride % 8 == 0 && y_row_stride % 4 == 0,
              TRIDA_ERR_ARG, "skinny_gemm: bad strides");
  TRIDA_CHECK(((((uintptr_t)X) | (uintptr_t)W) & 15) == 0 && ((uintptr_t)Y & 7) == 0, TRIDA_ERR_ALIGN,
              "skinny_gemm: X and W 16-byte aligned, Y 8-byte aligned");
  const int sk = plan_sk(N, K, splits);
  TRIDA_CHECK(sk >= 1 && sk <= 65535 && N / 16 < INT32_MAX, TRIDA_ERR_ARG, "skinny_gemm: bad split count");
  TRIDA_CHECK(sk == 1 || (scratch && scratch_bytes >= trida_skinny_gemm_scratch_bytes(M, N, K, sk)), TRIDA_ERR_WORKSPACE,
              "skinny_gemm: scratch too small for %d K splits", sk);
  GemmArgs a{X, W, Y, static_cast<float*>(scratch), x_row_stride, w_row_stride, y_row_stride, (int)M, (int)N,
             (int)K, sk};
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)(N / 16), (unsigned)sk);
  const int mt = (int)cdiv(M, 16);
  switch (mt) {
    case 1: hipLaunchKernelGGL(skinny_gemm_kernel<1>, grid, dim3(kNW * kWave), 0, st, a); break;
    case 2: hipLaunchKernelGGL(skinny_gemm_kernel<2>, grid, dim3(kNW * kWave), 0, st, a); break;
    case 3: hipLaunchKernelGGL(skinny_gemm_kernel<3>, grid, dim3(kNW * kWave), 0, st, a); break;
    default: hipLaunchKernelGGL(skinny_gemm_kernel<4>, grid, dim3(kNW * kWave), 0, st, a); break;
  }
  int rc = launch_status("skinny_gemm");
  if (rc || sk == 1) return rc;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)cdiv(M * N / 4, 256)), dim3(256), 0, st,
                     static_cast<const float*>(scratch), Y, y_row_stride, (int)M, (int)N, sk);
  return launch_status("skinny_gemm/reduce");
}
