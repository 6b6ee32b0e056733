// Skinny bf16 GEMM for the decode-step projections: Y[M, N] = X[M, K] W[N, K]^T with M <= 64
// (a canvas of <= 64 rows), fp32 accumulation, bf16 output. At these M the GEMM is bound by the weight
// stream, so the kernel is built to read every weight byte exactly once, with enough of them in flight
// to cover the HBM latency:
//   - v_mfma_f32_16x16x32_bf16 accumulates C^T[n, m]: the weight rows are the A operand (16-byte
//     loads straight into registers; plain loads: the nontemporal hint measured 15-30% slower on a
//     pure weight stream), the activation rows the B operand (L2-resident);
//   - a wave owns NR tiles of 16 weight rows, so each activation fragment it loads feeds NR MFMAs,
//     and issues KU k-steps of loads (NR * KU weight fragments) before the MFMAs that consume them;
//   - the NW waves of a workgroup split K and reduce through LDS; NR and NW are chosen per shape so
//     that the grid holds ~1000 or more waves without splitting K across workgroups (which would cost
//     fp32 partials and a reduce launch; kept for shapes too narrow for that).
// Each output's K sum runs in an order that depends on N and K only, so a row of Y is the same whether
// X holds 1 row or 64.
#include <algorithm>

#include "common.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ bf16x8 as_bf(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

struct GemmArgs {
  const uint16_t* X;
  const uint16_t* W;
  uint16_t* Y;
  float* partial;  // [SK, M, N] when SK > 1
  int64_t x_st, w_st, y_st;
  int M, N, K, SK;
};

template <int MT, int NR, int NW, int KU>
__global__ __launch_bounds__(NW* kWave) void skinny_gemm_kernel(GemmArgs a) {
  const int ng = blockIdx.x, sk = blockIdx.y;
  const int wave = threadIdx.x / kWave, l = threadIdx.x % kWave;
  const int ksteps = a.K / 32;
  const int part = sk * NW + wave, nparts = a.SK * NW;
  const int s0 = (int)((int64_t)ksteps * part / nparts);
  const int s1 = (int)((int64_t)ksteps * (part + 1) / nparts);
  const int n0 = ng * NR * 16;
  const u32x4* wrow[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r)
    wrow[r] = reinterpret_cast<const u32x4*>(a.W + (int64_t)(n0 + r * 16 + (l % 16)) * a.w_st + (l / 16) * 8);
  const u32x4* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = min(mt * 16 + (l % 16), a.M - 1);  // rows past M repeat the last row; never stored
    xrow[mt] = reinterpret_cast<const u32x4*>(a.X + (int64_t)m * a.x_st + (l / 16) * 8);
  }
  f32x4 acc[NR][MT];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[r][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  int s = s0;
  for (; s + KU <= s1; s += KU) {
    u32x4 wv[KU][NR];
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int r = 0; r < NR; ++r) wv[u][r] = wrow[r][(int64_t)(s + u) * 4];
    u32x4 xv[KU][MT];
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xv[u][mt] = xrow[mt][(int64_t)(s + u) * 4];
    // every load of the batch is issued before the first MFMA waits on one (the scheduler would
    // otherwise interleave them and keep only a few in flight)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < KU; ++u)
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(wv[u][r]), as_bf(xv[u][mt]), acc[r][mt], 0, 0, 0);
  }
  for (; s < s1; ++s) {
    u32x4 wv[NR], xv[MT];
#pragma unroll
    for (int r = 0; r < NR; ++r) wv[r] = wrow[r][(int64_t)s * 4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xv[mt] = xrow[mt][(int64_t)s * 4];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        acc[r][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(wv[r]), as_bf(xv[mt]), acc[r][mt], 0, 0, 0);
  }

  // reduce the NW waves' K parts; lane l holds C^T[n = (l/16)*4 + i][m = mt*16 + l%16] of each tile.
  // Waves 1.. park their partials, then wave w sums the tiles t = w, w + NW, ... and writes them.
  constexpr int NTILE = NR * MT;
  __shared__ f32x4 red[NW][NTILE][kWave];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][r * MT + mt][l] = acc[r][mt];
  __syncthreads();
  for (int t = wave; t < NTILE; t += NW) {
    f32x4 sum = red[0][t][l];
#pragma unroll
    for (int w = 1; w < NW; ++w) sum += red[w][t][l];
    const int r = t / MT, mt = t % MT;
    const int m = mt * 16 + (l % 16);
    if (m >= a.M) continue;
    const int n = n0 + r * 16 + (l / 16) * 4;
    if (a.SK == 1) {
      u32x2 packed;
      packed.x = f2bf2(sum.x, sum.y);
      packed.y = f2bf2(sum.z, sum.w);
      *reinterpret_cast<u32x2*>(a.Y + (int64_t)m * a.y_st + n) = packed;
    } else {
      *reinterpret_cast<f32x4*>(a.partial + ((int64_t)sk * a.M + m) * a.N + n) = sum;
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
  packed.x = f2bf2(s.x, s.y);
  packed.y = f2bf2(s.z, s.w);
  *reinterpret_cast<u32x2*>(Y + (int64_t)m * y_st + n) = packed;
}

// Launch plan from N and K only: rows per wave (NR tiles of 16), waves per workgroup splitting K (NW),
// k-steps in flight (KU) and K splits across workgroups (SK).
struct Plan {
  int nr, nw, ku, sk;
};
Plan plan(int64_t N, int64_t K, int64_t splits) {
  const int64_t tiles = N / 16, ksteps = K / 32;
  Plan p;
  if (tiles >= 1024 && N % 64 == 0) {
    p = {4, 4, 4, 1};
  } else if (tiles >= 512 && N % 32 == 0) {
    p = {2, 4, 8, 1};
  } else {
    p = {1, 8, 8, 1};
  }
  int64_t sk = splits > 0 ? splits : 1;
  if (splits <= 0) {
    const int64_t waves = tiles / p.nr * p.nw;
    if (waves < 512) sk = cdiv(512, waves);
  }
  const int64_t cap = std::max<int64_t>(1, ksteps / (p.nw * 2));  // at least ~2 k-steps per wave
  p.sk = (int)std::min<int64_t>(sk, cap);
  return p;
}

template <int MT, int NR, int NW, int KU>
void launch(const GemmArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)(a.N / (16 * NR)), (unsigned)a.SK);
  hipLaunchKernelGGL((skinny_gemm_kernel<MT, NR, NW, KU>), grid, dim3(NW * kWave), 0, st, a);
}
template <int MT>
void launch_mt(const GemmArgs& a, const Plan& p, hipStream_t st) {
  if (p.nr == 4) launch<MT, 4, 4, 4>(a, st);
  else if (p.nr == 2) launch<MT, 2, 4, 8>(a, st);
  else launch<MT, 1, 8, 8>(a, st);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_skinny_gemm_scratch_bytes(int64_t M, int64_t N, int64_t K, int64_t splits) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  const Plan p = plan(N, K, splits);
  return p.sk > 1 ? align_up((int64_t)p.sk * M * N * 4, 256) : 0;
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
  const Plan p = plan(N, K, splits);
  TRIDA_CHECK(p.sk >= 1 && p.sk <= 65535 && N / 16 < INT32_MAX, TRIDA_ERR_ARG, "skinny_gemm: bad split count");
  TRIDA_CHECK(p.sk == 1 || (scratch && scratch_bytes >= trida_skinny_gemm_scratch_bytes(M, N, K, splits)),
              TRIDA_ERR_WORKSPACE, "skinny_gemm: scratch too small for %d K splits", p.sk);
  GemmArgs a{X, W, Y, static_cast<float*>(scratch), x_row_stride, w_row_stride, y_row_stride, (int)M, (int)N,
             (int)K, p.sk};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch ((int)cdiv(M, 16)) {
    case 1: launch_mt<1>(a, p, st); break;
    case 2: launch_mt<2>(a, p, st); break;
    case 3: launch_mt<3>(a, p, st); break;
    default: launch_mt<4>(a, p, st); break;
  }
  int rc = launch_status("skinny_gemm");
  if (rc || p.sk == 1) return rc;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)cdiv(M * N / 4, 256)), dim3(256), 0, st,
                     static_cast<const float*>(scratch), Y, y_row_stride, (int)M, (int)N, p.sk);
  return launch_status("skinny_gemm/reduce");
}
