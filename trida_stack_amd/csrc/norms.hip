// Fused row-wise kernels of the hybrid decoder around the GEMMs (bf16 storage, fp32 arithmetic,
// one rounding per output):
//   add_rmsnorm    x = x + r (residual, in place), out = rmsnorm(x) * (1 + w)   (zero-centred weight)
//   silu_mul       out = silu(gu[:, :I]) * gu[:, I:]                            (SwiGLU)
//   gated_rmsnorm  out = bf16(o * rsqrt(mean(o^2) + eps)) * w * silu(z), per value head
//   attn_prep      per-head RMSNorm (zero-centred) of q and k, partial RoPE (rotate-half), q to a packed
//                  buffer, k and v into the KV cache at the sequence's device-side position
#include <math.h>

#include "common.h"

namespace trida {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void unpack8(const u32x4 w, float* f) {
  f[0] = bf2f((uint16_t)(w.x & 0xffff));
  f[1] = bf2f((uint16_t)(w.x >> 16));
  f[2] = bf2f((uint16_t)(w.y & 0xffff));
  f[3] = bf2f((uint16_t)(w.y >> 16));
  f[4] = bf2f((uint16_t)(w.z & 0xffff));
  f[5] = bf2f((uint16_t)(w.z >> 16));
  f[6] = bf2f((uint16_t)(w.w & 0xffff));
  f[7] = bf2f((uint16_t)(w.w >> 16));
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 w;
  w.x = f2bf2(f[0], f[1]);
  w.y = f2bf2(f[2], f[3]);
  w.z = f2bf2(f[4], f[5]);
  w.w = f2bf2(f[6], f[7]);
  return w;
}
__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }

__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / kWave, l = threadIdx.x % kWave;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) s += red[i];
  return s;
}

// ------------------------------------------------------------------ add + rmsnorm (one block per row)
constexpr int kMaxPieces = 4;  // 8 elements each per thread: dim <= 256 * 8 * 4 = 8192

// The residual r is either bf16 rows (r, r_st) or, with `parts`, the sum of n_parts fp32 planes of
// plane_st elements each (rows of dim floats): the split-K partial results of the weight-streaming GEMM,
// summed in plane order and rounded to bf16 as the GEMM's own output would be.
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(uint16_t* x, const uint16_t* r, const float* parts,
                                                               int n_parts, int64_t plane_st, const uint16_t* w,
                                                               uint16_t* out, int dim, int64_t x_st, int64_t r_st,
                                                               int64_t o_st, float eps, int zero_centred) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const int pieces = dim / 8;
  // every load (x, residual, weight) is issued before the reduction: one memory round trip per row
  u32x4 xr[kMaxPieces], rr[kMaxPieces], wr[kMaxPieces];
#pragma unroll
  for (int u = 0; u < kMaxPieces; ++u) {
    const int p = threadIdx.x + u * kThreads;
    if (p < pieces) {
      xr[u] = *reinterpret_cast<const u32x4*>(x + row * x_st + p * 8);
      if (r) rr[u] = *reinterpret_cast<const u32x4*>(r + row * r_st + p * 8);
      wr[u] = *reinterpret_cast<const u32x4*>(w + p * 8);
    }
  }
  if (parts) {
    float acc[kMaxPieces][8];
#pragma unroll
    for (int u = 0; u < kMaxPieces; ++u)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[u][j] = 0.f;
    for (int s = 0; s < n_parts; ++s) {
      const float* pl = parts + s * plane_st + row * dim;
#pragma unroll
      for (int u = 0; u < kMaxPieces; ++u) {
        const int p = threadIdx.x + u * kThreads;
        if (p < pieces) {
          const f32x4 a = *reinterpret_cast<const f32x4*>(pl + p * 8);
          const f32x4 b = *reinterpret_cast<const f32x4*>(pl + p * 8 + 4);
          acc[u][0] += a.x; acc[u][1] += a.y; acc[u][2] += a.z; acc[u][3] += a.w;
          acc[u][4] += b.x; acc[u][5] += b.y; acc[u][6] += b.z; acc[u][7] += b.w;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kMaxPieces; ++u) rr[u] = pack8(acc[u]);
  }
  const bool has_r = r || parts;  // its bf16 values are in rr
  float v[kMaxPieces][8];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxPieces; ++u) {
    const int p = threadIdx.x + u * kThreads;
    if (p < pieces) {
      unpack8(xr[u], v[u]);
      if (has_r) {
        float rv[8];
        unpack8(rr[u], rv);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[u][j] = bf2f(f2bf(v[u][j] + rv[j]));  // the residual stream is bf16
        *reinterpret_cast<u32x4*>(x + row * x_st + p * 8) = pack8(v[u]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[u][j], v[u][j], ss);
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / dim + eps);
#pragma unroll
  for (int u = 0; u < kMaxPieces; ++u) {
    const int p = threadIdx.x + u * kThreads;
    if (p < pieces) {
      float wv[8], y[8];
      unpack8(wr[u], wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = v[u][j] * inv * (zero_centred ? 1.f + wv[j] : wv[j]);
      *reinterpret_cast<u32x4*>(out + row * o_st + p * 8) = pack8(y);
    }
  }
}

// ------------------------------------------------------------------ silu(g) * u
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const uint16_t* gu, uint16_t* out, int inter,
                                                            int64_t g_st, int64_t o_st, int64_t n_pieces) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n_pieces) return;
  const int per_row = inter / 8;
  const int64_t row = i / per_row;
  const int c = (int)(i % per_row) * 8;
  float g[8], u[8], y[8];
  unpack8(*reinterpret_cast<const u32x4*>(gu + row * g_st + c), g);
  unpack8(*reinterpret_cast<const u32x4*>(gu + row * g_st + inter + c), u);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[j] = silu(g[j]) * u[j];
  *reinterpret_cast<u32x4*>(out + row * o_st + c) = pack8(y);
}

// ------------------------------------------------------------------ gated rmsnorm (one wave per (row, head))
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(const uint16_t* o, const uint16_t* z,
                                                                 const uint16_t* w, uint16_t* out, int64_t rows,
                                                                 int H, int Dv, int64_t z_st, float eps) {
  const int64_t gw = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (gw >= rows * H) return;
  const int l = threadIdx.x % kWave;
  const int64_t row = gw / H;
  const int h = (int)(gw % H);
  const int per = Dv / kWave;  // elements per lane (Dv in {64, 128, 256})
  const uint16_t* op = o + (row * H + h) * Dv + l * per;
  const uint16_t* zp = z + row * z_st + (int64_t)h * Dv + l * per;
  // o, gate and weight are all loaded before the reduction: one memory round trip
  float v[4], zv[4], wv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < per) {
      v[j] = bf2f(op[j]);
      zv[j] = bf2f(zp[j]);
      wv[j] = bf2f(w[l * per + j]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j < per) ss = fmaf(v[j], v[j], ss);
  const float inv = rsqrtf(wave_sum(ss) / Dv + eps);
  uint16_t* dst = out + (row * H + h) * Dv + l * per;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < per) {
      const float nrm = bf2f(f2bf(v[j] * inv));  // normalised value in the input dtype, then weight and gate
      dst[j] = f2bf(nrm * wv[j] * silu(zv[j]));
    }
  }
}

// ------------------------------------------------------------------ attention prep (one wave per (row, head))
struct AttnPrepArgs {
  const uint16_t* qkv;  // row (b, t): [Hq x (q D | gate D)] [Hkv x k D] [Hkv x v D], row stride qkv_st
  const uint16_t* qn_w;  // [D] zero-centred
  const uint16_t* kn_w;
  const int32_t* pos0;    // [B] position of row 0 (RoPE)
  const int32_t* slot0;   // [B] cache slot of row 0
  uint16_t* q_out;        // [B, T, Hq, D]
  uint16_t* k_cache;      // [B, Hkv, Lmax, D]
  uint16_t* v_cache;
  int T, Hq, Hkv, D, Lmax, rot;
  int64_t qkv_st;
  float eps, log2_theta;
};

__global__ __launch_bounds__(kThreads) void attn_prep_kernel(AttnPrepArgs a) {
  constexpr int kMaxPer = 4;  // D <= 256
  const int heads = a.Hq + 2 * a.Hkv;
  const int bb = blockIdx.y;  // sequence
  const int64_t gw = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;  // (t, head) of bb
  if (gw >= (int64_t)a.T * heads) return;  // whole waves exit together
  const int l = threadIdx.x % kWave;
  const int t = (int)(gw / heads), hh = (int)(gw % heads);
  const int per = a.D / kWave;
  const uint16_t* row = a.qkv + ((int64_t)bb * a.T + t) * a.qkv_st;
  const uint16_t* src;
  int kind;  // 0 q, 1 k, 2 v
  int h;
  if (hh < a.Hq) {
    kind = 0;
    h = hh;
    src = row + (int64_t)h * 2 * a.D;
  } else if (hh < a.Hq + a.Hkv) {
    kind = 1;
    h = hh - a.Hq;
    src = row + (int64_t)a.Hq * 2 * a.D + (int64_t)h * a.D;
  } else {
    kind = 2;
    h = hh - a.Hq - a.Hkv;
    src = row + (int64_t)a.Hq * 2 * a.D + (int64_t)a.Hkv * a.D + (int64_t)h * a.D;
  }
  float v[kMaxPer], wnv[kMaxPer];
  const uint16_t* wn = kind == 0 ? a.qn_w : a.kn_w;  // loaded with the row: one memory round trip
  for (int j = 0; j < per; ++j) {
    v[j] = bf2f(src[l * per + j]);
    wnv[j] = bf2f(wn[l * per + j]);
  }
  const int64_t slot = (int64_t)a.slot0[bb] + t;
  // rows past the cache capacity (a caller's overlong decode) write no K / V (one (t, head) per wave,
  // so the whole wave leaves together)
  if (kind != 0 && (slot < 0 || slot >= a.Lmax)) return;
  if (kind == 2) {
    uint16_t* dst = a.v_cache + (((int64_t)bb * a.Hkv + h) * a.Lmax + slot) * a.D + l * per;
    for (int j = 0; j < per; ++j) dst[j] = f2bf(v[j]);
    return;
  }
  float ss = 0.f;
  for (int j = 0; j < per; ++j) ss = fmaf(v[j], v[j], ss);
  const float inv = rsqrtf(wave_sum(ss) / a.D + a.eps);
  for (int j = 0; j < per; ++j) v[j] = bf2f(f2bf(v[j] * inv * (1.f + wnv[j])));
  // partial rotary (rotate-half over the first `rot` dims): x1 = [0, rot/2), x2 = [rot/2, rot).
  // half is a multiple of the per-lane width, so a lane's partner values sit in one other lane.
  const int half = a.rot / 2;
  const int shift = half / per;
  const bool first = l * per < half;
  const int partner = first ? l + shift : l - shift;
  const float pos = (float)(a.pos0[bb] + t);
  float y[kMaxPer];
  for (int j = 0; j < per; ++j) {
    const int d = l * per + j;
    const float other = __shfl(v[j], partner < kWave ? partner : l, kWave);
    y[j] = v[j];
    if (d < a.rot) {
      const int i = first ? d : d - half;
      const float inv_freq = exp2f(-a.log2_theta * (2.f * i) / a.rot);  // theta^(-2i / rot)
      float sn, cs;
      sincosf(pos * inv_freq, &sn, &cs);
      y[j] = first ? v[j] * cs - other * sn : v[j] * cs + other * sn;
    }
  }
  uint16_t* dst = kind == 0 ? a.q_out + (((int64_t)bb * a.T + t) * a.Hq + h) * a.D + l * per
                            : a.k_cache + (((int64_t)bb * a.Hkv + h) * a.Lmax + slot) * a.D + l * per;
  for (int j = 0; j < per; ++j) dst[j] = f2bf(y[j]);
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_add_rmsnorm(uint16_t* x, const uint16_t* r, const uint16_t* w, uint16_t* out, int64_t rows,
                                 int64_t dim, int64_t x_st, int64_t r_st, int64_t o_st, float eps, int zero_centred,
                                 void* stream) {
  TRIDA_CHECK(x && w && out, TRIDA_ERR_NULL, "add_rmsnorm: x, w and out are required");
  TRIDA_CHECK(rows > 0 && dim > 0 && dim % 8 == 0 && dim <= kThreads * 8 * kMaxPieces, TRIDA_ERR_ARG,
              "add_rmsnorm: dim must be a multiple of 8 and <= %d", kThreads * 8 * kMaxPieces);
  TRIDA_CHECK(x_st % 8 == 0 && r_st % 8 == 0 && o_st % 8 == 0 &&
                  ((((uintptr_t)x) | (uintptr_t)r | (uintptr_t)w | (uintptr_t)out) & 15) == 0,
              TRIDA_ERR_ALIGN, "add_rmsnorm: 16-byte aligned rows required");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     x, r, static_cast<const float*>(nullptr), 0, (int64_t)0, w, out, (int)dim, x_st, r_st, o_st, eps,
                     zero_centred);
  return launch_status("add_rmsnorm");
}

extern "C" int trida_add_rmsnorm_parts(uint16_t* x, const float* parts, int64_t n_parts, int64_t plane_stride,
                                       const uint16_t* w, uint16_t* out, int64_t rows, int64_t dim, int64_t x_st,
                                       int64_t o_st, float eps, int zero_centred, void* stream) {
  TRIDA_CHECK(x && parts && w && out, TRIDA_ERR_NULL, "add_rmsnorm_parts: x, parts, w and out are required");
  TRIDA_CHECK(rows > 0 && rows < 65536 && dim > 0 && dim % 8 == 0 && dim <= kThreads * 8 * kMaxPieces &&
                  n_parts >= 1 && n_parts <= 64 && plane_stride >= rows * dim,
              TRIDA_ERR_ARG, "add_rmsnorm_parts: bad sizes (dim a multiple of 8 <= %d, 1 <= n_parts <= 64)",
              kThreads * 8 * kMaxPieces);
  TRIDA_CHECK(x_st % 8 == 0 && o_st % 8 == 0 && plane_stride % 4 == 0 &&
                  ((((uintptr_t)x) | (uintptr_t)parts | (uintptr_t)w | (uintptr_t)out) & 15) == 0,
              TRIDA_ERR_ALIGN, "add_rmsnorm_parts: 16-byte aligned rows required");
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     x, static_cast<const uint16_t*>(nullptr), parts, (int)n_parts, plane_stride, w, out, (int)dim, x_st,
                     (int64_t)0, o_st, eps, zero_centred);
  return launch_status("add_rmsnorm_parts");
}

extern "C" int trida_silu_mul(const uint16_t* gu, uint16_t* out, int64_t rows, int64_t inter, int64_t g_st,
                              int64_t o_st, void* stream) {
  TRIDA_CHECK(gu && out, TRIDA_ERR_NULL, "silu_mul: gu and out are required");
  TRIDA_CHECK(rows > 0 && inter > 0 && inter % 8 == 0 && g_st >= 2 * inter && g_st % 8 == 0 && o_st % 8 == 0,
              TRIDA_ERR_ARG, "silu_mul: bad sizes");
  TRIDA_CHECK(((((uintptr_t)gu) | (uintptr_t)out) & 15) == 0, TRIDA_ERR_ALIGN, "silu_mul: alignment");
  const int64_t n = rows * (inter / 8);
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)cdiv(n, kThreads)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), gu, out, (int)inter, g_st, o_st, n);
  return launch_status("silu_mul");
}

extern "C" int trida_gated_rmsnorm(const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out,
                                   int64_t rows, int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream) {
  TRIDA_CHECK(o && z && w && out, TRIDA_ERR_NULL, "gated_rmsnorm: o, z, w and out are required");
  TRIDA_CHECK(rows > 0 && H > 0 && (Dv == 64 || Dv == 128 || Dv == 256) && z_st >= H * Dv, TRIDA_ERR_ARG,
              "gated_rmsnorm: Dv must be 64, 128 or 256");
  const int64_t waves = rows * H;
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3((unsigned)cdiv(waves, kThreads / kWave)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), o, z, w, out, rows, (int)H, (int)Dv, z_st, eps);
  return launch_status("gated_rmsnorm");
}

extern "C" int trida_attn_prep(const uint16_t* qkv, int64_t qkv_row_stride, const uint16_t* q_norm_w,
                               const uint16_t* k_norm_w, const int32_t* pos0, const int32_t* slot0, uint16_t* q_out,
                               uint16_t* k_cache, uint16_t* v_cache, int64_t B, int64_t T, int64_t Hq, int64_t Hkv,
                               int64_t D, int64_t Lmax, int64_t rot_dim, float rope_theta, float eps,
                               void* stream) {
  TRIDA_CHECK(qkv && q_norm_w && k_norm_w && pos0 && slot0 && q_out && k_cache && v_cache, TRIDA_ERR_NULL,
              "attn_prep: a required pointer is NULL");
  TRIDA_CHECK(B > 0 && B < 65536 && T > 0 && Hq > 0 && Hkv > 0 && (D == 64 || D == 128 || D == 256), TRIDA_ERR_ARG,
              "attn_prep: bad sizes");
  TRIDA_CHECK(rot_dim >= 0 && rot_dim <= D && rot_dim % 2 == 0, TRIDA_ERR_ARG, "attn_prep: bad rotary dim");
  TRIDA_CHECK(qkv_row_stride >= (2 * Hq + 2 * Hkv) * D, TRIDA_ERR_ARG, "attn_prep: qkv row stride too small");
  const int64_t waves = T * (Hq + 2 * Hkv);
  AttnPrepArgs a{qkv, q_norm_w, k_norm_w, pos0, slot0, q_out, k_cache, v_cache, (int)T, (int)Hq, (int)Hkv, (int)D,
                 (int)Lmax, (int)rot_dim, qkv_row_stride, eps, log2f(rope_theta)};
  hipLaunchKernelGGL(attn_prep_kernel, dim3((unsigned)cdiv(waves, kThreads / kWave), (unsigned)B), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status("attn_prep");
}
