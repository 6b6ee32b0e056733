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
// NU = pieces of 8 elements per thread (dim <= 2048 NU); MODE 0: no residual, 1: bf16 rows r, 2: fp32 planes.
// Every load is unconditional (the index clamped into the row; loads past it are dropped), so all of them
// are in flight together: one memory round trip per row.
template <int NU, int MODE>
__global__ __launch_bounds__(kThreads) void add_rmsnorm_kernel(uint16_t* x, const uint16_t* r, const float* parts,
                                                               int n_parts, int64_t plane_st, const uint16_t* w,
                                                               uint16_t* out, int dim, int64_t x_st, int64_t r_st,
                                                               int64_t o_st, float eps, int zero_centred) {
  __shared__ float red[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const int pieces = dim / 8;
  u32x4 xr[NU], rr[NU], wr[NU];
  f32x4 pv[MODE == 2 ? 8 : 1][NU][2];
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int p = min((int)threadIdx.x + u * kThreads, pieces - 1);
    if (MODE == 2) {
      const float* pl = parts + row * dim + p * 8;
#pragma unroll
      for (int s = 0; s < 8; ++s) {  // planes past n_parts re-read the last one and are dropped
        const float* q = pl + min(s, n_parts - 1) * plane_st;
        pv[s][u][0] = *reinterpret_cast<const f32x4*>(q);
        pv[s][u][1] = *reinterpret_cast<const f32x4*>(q + 4);
      }
    }
    xr[u] = *reinterpret_cast<const u32x4*>(x + row * x_st + p * 8);
    if (MODE == 1) rr[u] = *reinterpret_cast<const u32x4*>(r + row * r_st + p * 8);
    wr[u] = *reinterpret_cast<const u32x4*>(w + p * 8);
  }
  if (MODE == 2) {  // the planes summed in order and rounded to bf16, as the GEMM's own output would be
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int p = min((int)threadIdx.x + u * kThreads, pieces - 1);
      f32x4 a0 = pv[0][u][0], a1 = pv[0][u][1];
      const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 1; s < 8; ++s) {
        a0 += s < n_parts ? pv[s][u][0] : zero;
        a1 += s < n_parts ? pv[s][u][1] : zero;
      }
      for (int s = 8; s < n_parts; ++s) {
        const float* q = parts + s * plane_st + row * dim + p * 8;
        a0 += *reinterpret_cast<const f32x4*>(q);
        a1 += *reinterpret_cast<const f32x4*>(q + 4);
      }
      const float acc[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
      rr[u] = pack8(acc);
    }
  }
  float v[NU][8];
  float ss = 0.f;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int p = (int)threadIdx.x + u * kThreads;
    unpack8(xr[u], v[u]);
    if (MODE != 0) {
      float rv[8];
      unpack8(rr[u], rv);
#pragma unroll
      for (int j = 0; j < 8; ++j) v[u][j] = bf2f(f2bf(v[u][j] + rv[j]));  // the residual stream is bf16
      if (p < pieces) *reinterpret_cast<u32x4*>(x + row * x_st + p * 8) = pack8(v[u]);
    }
    if (p < pieces) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ss = fmaf(v[u][j], v[u][j], ss);
    }
  }
  const float inv = rsqrtf(block_sum(ss, red) / dim + eps);
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int p = (int)threadIdx.x + u * kThreads;
    if (p < pieces) {
      float wv[8], y[8];
      unpack8(wr[u], wv);
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = v[u][j] * inv * (zero_centred ? 1.f + wv[j] : wv[j]);
      *reinterpret_cast<u32x4*>(out + row * o_st + p * 8) = pack8(y);
    }
  }
}

template <int MODE>
void launch_add_rmsnorm(int64_t rows, int64_t dim, hipStream_t st, uint16_t* x, const uint16_t* r, const float* parts,
                        int n_parts, int64_t plane_st, const uint16_t* w, uint16_t* out, int64_t x_st, int64_t r_st,
                        int64_t o_st, float eps, int zero_centred) {
  const int nu = (int)cdiv(dim / 8, kThreads);
#define TRIDA_ARN(NU)                                                                                                 \
  hipLaunchKernelGGL((add_rmsnorm_kernel<NU, MODE>), dim3((unsigned)rows), dim3(kThreads), 0, st, x, r, parts, n_parts, \
                     plane_st, w, out, (int)dim, x_st, r_st, o_st, eps, zero_centred)
  switch (nu) {
    case 1: TRIDA_ARN(1); break;
    case 2: TRIDA_ARN(2); break;
    case 3: TRIDA_ARN(3); break;
    default: TRIDA_ARN(4); break;
  }
#undef TRIDA_ARN
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
// PER = Dv / 64 elements per lane, read as one vector per operand (o, gate, weight) before the reduction
// FRAG: out in the weight-streaming GEMM's fragment order (rows <= 48, K = H * Dv)
template <int PER, bool FRAG>
__global__ __launch_bounds__(kThreads) void gated_rmsnorm_kernel(const uint16_t* o, const uint16_t* z,
                                                                 const uint16_t* w, uint16_t* out, int64_t rows,
                                                                 int H, int64_t z_st, float eps) {
  constexpr int Dv = PER * kWave;
  const int64_t gw = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (gw >= rows * H) return;
  const int l = threadIdx.x % kWave;
  const int64_t row = gw / H;
  const int h = (int)(gw % H);
  const uint16_t* op = o + (row * H + h) * Dv + l * PER;
  const uint16_t* zp = z + row * z_st + (int64_t)h * Dv + l * PER;
  uint16_t ov[PER], zv[PER], wv[PER];
  if (PER == 4) {
    *reinterpret_cast<u32x2*>(ov) = *reinterpret_cast<const u32x2*>(op);
    *reinterpret_cast<u32x2*>(zv) = *reinterpret_cast<const u32x2*>(zp);
    *reinterpret_cast<u32x2*>(wv) = *reinterpret_cast<const u32x2*>(w + l * PER);
  } else if (PER == 2) {
    *reinterpret_cast<uint32_t*>(ov) = *reinterpret_cast<const uint32_t*>(op);
    *reinterpret_cast<uint32_t*>(zv) = *reinterpret_cast<const uint32_t*>(zp);
    *reinterpret_cast<uint32_t*>(wv) = *reinterpret_cast<const uint32_t*>(w + l * PER);
  } else {
    ov[0] = op[0];
    zv[0] = zp[0];
    wv[0] = w[l];
  }
  float v[PER], ss = 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    v[j] = bf2f(ov[j]);
    ss = fmaf(v[j], v[j], ss);
  }
  const float inv = rsqrtf(wave_sum(ss) / Dv + eps);
  uint16_t y[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const float nrm = bf2f(f2bf(v[j] * inv));  // normalised value in the input dtype, then weight and gate
    y[j] = f2bf(nrm * bf2f(wv[j]) * silu(bf2f(zv[j])));
  }
  uint16_t* dst = FRAG ? out + ws_frag_off((int)row, (int64_t)h * Dv + l * PER) : out + (row * H + h) * Dv + l * PER;
  if (PER == 4) *reinterpret_cast<u32x2*>(dst) = *reinterpret_cast<const u32x2*>(y);
  else if (PER == 2) *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(y);
  else dst[0] = y[0];
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

// kHG heads of one kind per wave: their rotary factors (one sincos per dim) are computed once. Large
// calls (batch 64) take 4 heads per wave; small ones (batch 1) 1, where more waves in flight matter more
template <int kHG>
__global__ __launch_bounds__(kThreads) void attn_prep_kernel(AttnPrepArgs a) {
  constexpr int kMaxPer = 4;  // D <= 256
  const int qg = (a.Hq + kHG - 1) / kHG, kg = (a.Hkv + kHG - 1) / kHG;
  const int groups = qg + 2 * kg;
  const int bb = blockIdx.y;  // sequence
  const int64_t gw = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;  // (t, head group) of bb
  if (gw >= (int64_t)a.T * groups) return;  // whole waves exit together
  const int l = threadIdx.x % kWave;
  const int t = (int)(gw / groups), gi = (int)(gw % groups);
  int kind, h0, nh;  // kind 0 q, 1 k, 2 v; heads h0 .. h0 + nh - 1
  if (gi < qg) {
    kind = 0;
    h0 = gi * kHG;
    nh = min(kHG, a.Hq - h0);
  } else if (gi < qg + kg) {
    kind = 1;
    h0 = (gi - qg) * kHG;
    nh = min(kHG, a.Hkv - h0);
  } else {
    kind = 2;
    h0 = (gi - qg - kg) * kHG;
    nh = min(kHG, a.Hkv - h0);
  }
  const int per = a.D / kWave;
  const int64_t slot = (int64_t)a.slot0[bb] + t;
  // rows past the cache capacity (a caller's overlong decode) write no K / V (uniform per wave)
  if (kind != 0 && (slot < 0 || slot >= a.Lmax)) return;
  const uint16_t* row = a.qkv + ((int64_t)bb * a.T + t) * a.qkv_st;
  const uint16_t* src0 = kind == 0 ? row : kind == 1 ? row + (int64_t)a.Hq * 2 * a.D
                                                     : row + (int64_t)a.Hq * 2 * a.D + (int64_t)a.Hkv * a.D;
  const int64_t hstride = kind == 0 ? 2 * a.D : a.D;  // q heads sit beside their output gates
  // every head of the group and the norm weights loaded together: one memory round trip. At D = 256 a
  // lane's 4 values move as one 8-byte piece when every row and pointer allows it (uniform per launch)
  const uint16_t* wn = kind == 0 ? a.qn_w : a.kn_w;
  const bool vec4 = per == 4 && (a.qkv_st & 3) == 0 &&
                    ((reinterpret_cast<uintptr_t>(a.qkv) | reinterpret_cast<uintptr_t>(wn) |
                      reinterpret_cast<uintptr_t>(a.q_out) | reinterpret_cast<uintptr_t>(a.k_cache) |
                      reinterpret_cast<uintptr_t>(a.v_cache)) & 7) == 0;
  auto load_row = [&](const uint16_t* p, float* f) {
    if (vec4) {
      const u32x2 w = *reinterpret_cast<const u32x2*>(p);
      f[0] = bf2f((uint16_t)(w.x & 0xffff));
      f[1] = bf2f((uint16_t)(w.x >> 16));
      f[2] = bf2f((uint16_t)(w.y & 0xffff));
      f[3] = bf2f((uint16_t)(w.y >> 16));
    } else {
#pragma unroll
      for (int j = 0; j < kMaxPer; ++j)
        if (j < per) f[j] = bf2f(p[j]);
    }
  };
  auto store_row = [&](uint16_t* p, const float* f) {
    if (vec4) {
      *reinterpret_cast<u32x2*>(p) = u32x2{f2bf2(f[0], f[1]), f2bf2(f[2], f[3])};
    } else {
#pragma unroll
      for (int j = 0; j < kMaxPer; ++j)
        if (j < per) p[j] = f2bf(f[j]);
    }
  };
  float v[kHG][kMaxPer], wnv[kMaxPer];
#pragma unroll
  for (int hh = 0; hh < kHG; ++hh) load_row(src0 + (int64_t)(h0 + (hh < nh ? hh : 0)) * hstride + l * per, v[hh]);
  load_row(wn + l * per, wnv);
  if (kind == 2) {
#pragma unroll
    for (int hh = 0; hh < kHG; ++hh) {
      if (hh < nh) store_row(a.v_cache + (((int64_t)bb * a.Hkv + h0 + hh) * a.Lmax + slot) * a.D + l * per, v[hh]);
    }
    return;
  }
  // partial rotary (rotate-half over the first `rot` dims): x1 = [0, rot/2), x2 = [rot/2, rot).
  // half is a multiple of the per-lane width, so a lane's partner values sit in one other lane. The
  // factors depend on the position and the dim only: one sincos per dim for the group's heads
  const int half = a.rot / 2;
  const int shift = half / per;
  const bool first = l * per < half;
  const int partner = first ? l + shift : l - shift;
  const float pos = (float)(a.pos0[bb] + t);
  float cs[kMaxPer], sn[kMaxPer];
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    cs[j] = 1.f;
    sn[j] = 0.f;
    const int d = l * per + j;
    if (j < per && d < a.rot) {
      const int i = first ? d : d - half;
      const float inv_freq = exp2f(-a.log2_theta * (2.f * i) / a.rot);  // theta^(-2i / rot)
      sincosf(pos * inv_freq, &sn[j], &cs[j]);
    }
  }
#pragma unroll
  for (int hh = 0; hh < kHG; ++hh) {
    if (hh < nh) {  // uniform
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxPer; ++j)
        if (j < per) ss = fmaf(v[hh][j], v[hh][j], ss);
      const float inv = rsqrtf(wave_sum(ss) / a.D + a.eps);
#pragma unroll
      for (int j = 0; j < kMaxPer; ++j)
        if (j < per) v[hh][j] = bf2f(f2bf(v[hh][j] * inv * (1.f + wnv[j])));
      float y[kMaxPer];
#pragma unroll
      for (int j = 0; j < kMaxPer; ++j) {
        if (j < per) {
          const int d = l * per + j;
          const float other = __shfl(v[hh][j], partner < kWave ? partner : l, kWave);
          y[j] = v[hh][j];
          if (d < a.rot) y[j] = first ? v[hh][j] * cs[j] - other * sn[j] : v[hh][j] * cs[j] + other * sn[j];
        }
      }
      store_row(kind == 0 ? a.q_out + (((int64_t)bb * a.T + t) * a.Hq + h0 + hh) * a.D + l * per
                          : a.k_cache + (((int64_t)bb * a.Hkv + h0 + hh) * a.Lmax + slot) * a.D + l * per,
                y);
    }
  }
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
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (r)
    launch_add_rmsnorm<1>(rows, dim, st, x, r, nullptr, 0, 0, w, out, x_st, r_st, o_st, eps, zero_centred);
  else
    launch_add_rmsnorm<0>(rows, dim, st, x, r, nullptr, 0, 0, w, out, x_st, r_st, o_st, eps, zero_centred);
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
  launch_add_rmsnorm<2>(rows, dim, static_cast<hipStream_t>(stream), x, nullptr, parts, (int)n_parts, plane_stride, w,
                        out, x_st, 0, o_st, eps, zero_centred);
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

namespace {
int gated_rmsnorm_run(const char* name, const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out,
                      bool frag, int64_t rows, int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream) {
  TRIDA_CHECK(o && z && w && out, TRIDA_ERR_NULL, "%s: o, z, w and out are required", name);
  TRIDA_CHECK(rows > 0 && H > 0 && (Dv == 64 || Dv == 128 || Dv == 256) && z_st >= H * Dv, TRIDA_ERR_ARG,
              "%s: Dv must be 64, 128 or 256", name);
  TRIDA_CHECK(!frag || (rows <= 48 && ((uintptr_t)out & 15) == 0), TRIDA_ERR_ARG,
              "%s: the fragment order holds at most 48 rows (16-byte aligned)", name);
  const int64_t waves = rows * H;
  const dim3 grid((unsigned)cdiv(waves, kThreads / kWave));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per = Dv / kWave;  // elements per lane, read as one vector of 2 * per bytes
  TRIDA_CHECK(((((uintptr_t)o) | (uintptr_t)z | (uintptr_t)w | (uintptr_t)out) & (2 * per - 1)) == 0 && z_st % per == 0,
              TRIDA_ERR_ALIGN, "%s: rows aligned to 2 * Dv / 64 bytes required", name);
#define TRIDA_GRN(PER)                                                                                              \
  if (frag)                                                                                                         \
    hipLaunchKernelGGL((gated_rmsnorm_kernel<PER, true>), grid, dim3(kThreads), 0, st, o, z, w, out, rows, (int)H,  \
                       z_st, eps);                                                                                  \
  else                                                                                                              \
    hipLaunchKernelGGL((gated_rmsnorm_kernel<PER, false>), grid, dim3(kThreads), 0, st, o, z, w, out, rows, (int)H, \
                       z_st, eps);
  if (Dv == 256) {
    TRIDA_GRN(4)
  } else if (Dv == 128) {
    TRIDA_GRN(2)
  } else {
    TRIDA_GRN(1)
  }
#undef TRIDA_GRN
  return launch_status(name);
}
}  // namespace

extern "C" int trida_gated_rmsnorm(const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out,
                                   int64_t rows, int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream) {
  return gated_rmsnorm_run("gated_rmsnorm", o, z, w, out, false, rows, H, Dv, z_st, eps, stream);
}

extern "C" int trida_gated_rmsnorm_frag(const uint16_t* o, const uint16_t* z, const uint16_t* w, uint16_t* out_frag,
                                        int64_t rows, int64_t H, int64_t Dv, int64_t z_st, float eps, void* stream) {
  return gated_rmsnorm_run("gated_rmsnorm_frag", o, z, w, out_frag, true, rows, H, Dv, z_st, eps, stream);
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
  const int hg = B * T >= 512 ? 4 : 1;  // heads per wave
  const int64_t waves = T * (cdiv(Hq, hg) + 2 * cdiv(Hkv, hg));  // (row, group of hg heads of one kind)
  AttnPrepArgs a{qkv, q_norm_w, k_norm_w, pos0, slot0, q_out, k_cache, v_cache, (int)T, (int)Hq, (int)Hkv, (int)D,
                 (int)Lmax, (int)rot_dim, qkv_row_stride, eps, log2f(rope_theta)};
  const dim3 grid((unsigned)cdiv(waves, kThreads / kWave), (unsigned)B);
  if (hg == 4) hipLaunchKernelGGL(attn_prep_kernel<4>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  else hipLaunchKernelGGL(attn_prep_kernel<1>, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), a);
  return launch_status("attn_prep");
}
