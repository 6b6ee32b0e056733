// GDN layer front half, fused: depthwise causal conv (width Kc) over [window ++ x] + SiLU, split
// into q / k / v, l2norm of q and k per head, and the gates g = -exp(A_log) softplus(a + dt_bias),
// beta = sigmoid(b).
//
// Launch: small grids take a grid of (sequence, row) x channel slices of 128 pieces (the C = conv_dim
// channels of a row spread over several CUs; at batch 1 a row per block would leave most of the GPU idle
// while each block pulls its 4 source rows and the whole conv weight); grids of >= 512 rows, which fill
// the GPU anyway, one 256-thread block per row with up to 4 passes over its pieces. A thread owns 8
// consecutive channels (one 16-byte piece) per pass; the Dk/8 threads of a q or k head reduce its sum of
// squares with a row-local reduction.
// Rounding follows the CPU oracle: conv and SiLU in fp32, rounded to bf16, then l2norm in fp32 of the
// rounded values, rounded to bf16 again.
#include "common.h"

namespace trida {
namespace {

constexpr int kMaxKc = 4;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  // update_dpp with a defined old value and bound_ctrl: folds into the consuming add / max
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
// Sum over aligned groups of W lanes (W = 4, 8 or 16); every lane receives its group's total.
template <int W>
__device__ __forceinline__ float lane_group_sum(float v) {
  if (W == 16) {
    v += dpp<0x128>(v);
    v += dpp<0x124>(v);
  } else if (W == 8) {
    v += __shfl_xor(v, 4, kWave);
  }
  v += dpp<0x4E>(v);
  v += dpp<0xB1>(v);
  return v;
}

struct PrepArgs {
  const uint16_t* x;  // [B, T, C] (batch stride x_sb, row stride x_st)
  const uint16_t* window;  // [B, Kc-1, C]
  const uint16_t* conv_w;  // [C, Kc]
  const uint16_t* a_in;    // [B, T, Hv] (batch stride ab_sb, row stride ab_st)
  const uint16_t* b_in;
  const float* A_log;  // [Hv]
  const float* dt_bias;
  uint16_t* q;  // [B, T, Hk, Dk]
  uint16_t* k;
  uint16_t* v;  // [B, T, Hv, Dv]
  float* g;     // [B, T, Hv]
  float* beta;
  uint16_t* window_out;  // [B, Kc-1, C] or null
  uint16_t* pre_out;     // [B, T, C] copy of the pre-conv rows x, or null
  const uint16_t* conv_bias;   // [C] or null
  const int32_t* win_idx;      // [B] window / window_out row of sequence b, or null (row b)
  const int32_t* pre_idx;      // [B] pre_out slot of sequence b, or null (slot b)
  const int32_t* cu_seqlens;   // [B + 1] packed ragged rows, or null (B x T rows)
  int T, C, Kc, Hk, Hv, Dk, Dv;
  int64_t x_sb, x_st, ab_sb, ab_st;
};

// Rows of sequence b: [row0, row0 + n) of the packed arrays. Contiguous form: n = T, row0 = b T (x and
// a / b rows then also move by their batch strides). Packed form: rows cu[b] .. cu[b + 1] - 1, at most T.
struct SeqRows {
  int64_t row0;
  int n;
};
__device__ __forceinline__ SeqRows seq_rows(const int32_t* cu_seqlens, int T, int b) {
  if (!cu_seqlens) return {(int64_t)b * T, T};
  const int lo = cu_seqlens[b];
  return {lo, max(0, min(cu_seqlens[b + 1] - lo, T))};
}

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
// torch.nn.functional.softplus with beta 1 and threshold 20
__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(__expf(x)); }

// IDX: the pool / packed forms (slot indices, cu_seqlens) may be in use; without it those pointers are ignored
// (null) and the plain form compiles without their loads and branches.
template <int GW, int KC, int NT, int PASSES, bool IDX>  // lanes per q/k head = Dk / 8; conv width; threads; passes
__global__ __launch_bounds__(NT) void gdn_prep_kernel(PrepArgs a) {
  const int32_t* cu_seqlens = IDX ? a.cu_seqlens : nullptr;
  const int32_t* win_idx = IDX ? a.win_idx : nullptr;
  const int32_t* pre_idx = IDX ? a.pre_idx : nullptr;
  const int t = blockIdx.x % a.T;
  const int b = blockIdx.x / a.T;
  const SeqRows sr = seq_rows(cu_seqlens, a.T, b);
  if (t >= sr.n) return;  // past a packed sequence's rows (block-uniform)
  const int T = sr.n;
  const int tid = threadIdx.x;
  const int key_dim = a.Hk * a.Dk;
  const int pieces = a.C / 8;
  const int pbase = blockIdx.y * NT * PASSES;  // the block's first piece: a multiple of GW
  // the sequence's source rows (packed: row r of x at r x_st) and its window row
  const uint16_t* xb = cu_seqlens ? a.x + sr.row0 * a.x_st : a.x + (int64_t)b * a.x_sb;
  const int64_t ab0 = cu_seqlens ? sr.row0 * a.ab_st : (int64_t)b * a.ab_sb;
  const int wrow = win_idx ? win_idx[b] : b;
  const int prow_b = pre_idx ? pre_idx[b] : b;  // pre_out slot
  const uint16_t* wb = a.window + (int64_t)wrow * (a.Kc - 1) * a.C;
  const int64_t orow = sr.row0 + t;  // output row (q, k, v, g, beta)

  // every load of the block first (one memory round trip): the gate inputs, then per pass the KC source rows
  // of the thread's 8 channels, their conv weights (8 channels x KC taps, contiguous: KC 16-byte pieces) and
  // bias. The loads are unconditional (the gate inputs of blocks that do not write the gates, the bias from
  // the conv weights when there is none: in bounds, unused), so that no branch splits the round trip. Lanes
  // past the last piece load it (clamped) and store nothing; passes past it are skipped (block-uniform)
  const bool gates = blockIdx.y == 0;  // block-uniform
  const int hg = min(tid, a.Hv - 1);
  const uint16_t ar = a.a_in[ab0 + (int64_t)t * a.ab_st + hg];
  const uint16_t br = a.b_in[ab0 + (int64_t)t * a.ab_st + hg];
  const float alog = a.A_log[hg], dtb = a.dt_bias[hg];
  const uint16_t* cbias = a.conv_bias ? a.conv_bias : a.conv_w;
  u32x4 xs[PASSES][KC], wsv[PASSES][KC], bsv[PASSES];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    if (pbase + ps * NT >= pieces) break;
    const int c = min(pbase + ps * NT + tid, pieces - 1) * 8;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int tau = t - (KC - 1) + j;  // source row; negative rows come from the window
      const uint16_t* src = tau >= 0 ? xb + (int64_t)tau * a.x_st + c : wb + (int64_t)(KC - 1 + tau) * a.C + c;
      xs[ps][j] = *reinterpret_cast<const u32x4*>(src);
      wsv[ps][j] = reinterpret_cast<const u32x4*>(a.conv_w + (int64_t)c * KC)[j];
    }
    bsv[ps] = *reinterpret_cast<const u32x4*>(cbias + c);
  }
  float av = bf2f(ar), bv = bf2f(br);

#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int p0 = pbase + ps * NT;
    if (p0 >= pieces) break;  // uniform
    const int p = p0 + tid;
    const bool live = p < pieces;
    const int c = min(p, pieces - 1) * 8;
    // the pre-conv rows a rollback rebuilds the window from: the block's own row is its last source row
    if (a.pre_out && live) {
      const int64_t prow = (int64_t)prow_b * a.T + t;
      *reinterpret_cast<u32x4*>(a.pre_out + prow * a.C + c) = xs[ps][KC - 1];
    }
    float acc[8];
    {
      float w[8][KC];
#pragma unroll
      for (int ch = 0; ch < 8; ++ch)
#pragma unroll
        for (int j = 0; j < KC; ++j) {
          const int e = ch * KC + j;  // element of the 8 x KC weight block
          const uint32_t word = wsv[ps][e / 8][(e % 8) / 2];
          w[ch][j] = __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
        }
      float bias[8];
      unpack8(bsv[ps], bias);
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) acc[ch] = a.conv_bias ? bias[ch] : 0.f;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        float f[8];
        unpack8(xs[ps][j], f);
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) acc[ch] = fmaf(w[ch][j], f[ch], acc[ch]);
      }
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) acc[ch] = bf2f(f2bf(silu(acc[ch])));
    }
    // the q/k pieces come first (2 * key_dim / 8 of them, a multiple of GW) and are all live, so every
    // group of GW lanes belongs to one head
    if (p0 < 2 * key_dim / 8) {  // block-uniform: per-head l2norm (all lanes take part in the reduction)
      const bool is_qk = c < 2 * key_dim;  // uniform across a GW-lane group
      float ss = 0.f;
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) ss = fmaf(acc[ch], acc[ch], ss);
      ss = lane_group_sum<GW>(ss);
      if (is_qk) {
        const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) acc[ch] *= inv;
      }
    }
    if (live) {
      const u32x4 w = pack8(acc);
      const int64_t row = orow;
      if (c < key_dim)
        *reinterpret_cast<u32x4*>(a.q + row * key_dim + c) = w;
      else if (c < 2 * key_dim)
        *reinterpret_cast<u32x4*>(a.k + row * key_dim + (c - key_dim)) = w;
      else
        *reinterpret_cast<u32x4*>(a.v + row * (int64_t)a.Hv * a.Dv + (c - 2 * key_dim)) = w;
    }
    // the new conv window (last Kc-1 rows of [window ++ x]): the last row's blocks, each its own pieces
    if (a.window_out && t == T - 1 && live) {
      for (int wr = 0; wr < a.Kc - 1; ++wr) {
        const int tau = T - (a.Kc - 1) + wr;
        const uint16_t* src = tau >= 0 ? xb + (int64_t)tau * a.x_st + c : wb + (int64_t)(a.Kc - 1 + tau) * a.C + c;
        *reinterpret_cast<u32x4*>(a.window_out + ((int64_t)wrow * (a.Kc - 1) + wr) * a.C + c) =
            *reinterpret_cast<const u32x4*>(src);
      }
    }
  }
  if (gates) {
    for (int hh = tid; hh < a.Hv; hh += NT) {
      if (hh != tid) {  // more heads than threads: the later ones load their own inputs
        av = bf2f(a.a_in[ab0 + (int64_t)t * a.ab_st + hh]);
        bv = bf2f(a.b_in[ab0 + (int64_t)t * a.ab_st + hh]);
      }
      const int64_t o = orow * a.Hv + hh;
      a.g[o] = -__expf(hh == tid ? alog : a.A_log[hh]) * softplus(av + (hh == tid ? dtb : a.dt_bias[hh]));
      a.beta[o] = 1.f / (1.f + __expf(-bv));
    }
  }
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_gdn_prep(const uint16_t* x, const uint16_t* window, const uint16_t* conv_w,
                              const uint16_t* a_in, const uint16_t* b_in, const float* A_log,
                              const float* dt_bias, uint16_t* q, uint16_t* k, uint16_t* v, float* g,
                              float* beta, uint16_t* window_out, uint16_t* pre_out, int64_t B, int64_t T, int64_t Kc,
                              int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv, int64_t x_sb, int64_t x_st,
                              int64_t ab_sb, int64_t ab_st, const uint16_t* conv_bias, const int32_t* win_idx,
                              const int32_t* pre_idx, const int32_t* cu_seqlens, void* stream) {
  TRIDA_CHECK(x && window && conv_w && a_in && b_in && A_log && dt_bias && q && k && v && g && beta,
              TRIDA_ERR_NULL, "gdn_prep: a required pointer is NULL");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0 && Kc >= 2 && Kc <= kMaxKc, TRIDA_ERR_ARG,
              "gdn_prep: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld Kc=%lld", (long long)B, (long long)T,
              (long long)Hk, (long long)Hv, (long long)Kc);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128, TRIDA_ERR_ARG, "gdn_prep: Dk must be 32, 64 or 128");
  TRIDA_CHECK(Dv % 8 == 0, TRIDA_ERR_ARG, "gdn_prep: Dv %% 8 == 0 required");
  const int64_t C = 2 * Hk * Dk + Hv * Dv;
  TRIDA_CHECK(x_st % 8 == 0 && x_sb % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)window & 15) == 0,
              TRIDA_ERR_ALIGN, "gdn_prep: x / window must be 16-byte aligned with strides in multiples of 8");
  TRIDA_CHECK(x_st >= C, TRIDA_ERR_ARG, "gdn_prep: row stride of x smaller than conv_dim");
  TRIDA_CHECK(((uintptr_t)conv_w & 15) == 0, TRIDA_ERR_ALIGN, "gdn_prep: conv_w must be 16-byte aligned");
  TRIDA_CHECK(window_out == nullptr || window_out != window, TRIDA_ERR_ARG,
              "gdn_prep: window_out must not alias window");
  TRIDA_CHECK(pre_out == nullptr || (((uintptr_t)pre_out & 15) == 0 && pre_out != x), TRIDA_ERR_ARG,
              "gdn_prep: pre_out must be 16-byte aligned and not alias x");
  TRIDA_CHECK(conv_bias == nullptr || ((uintptr_t)conv_bias & 15) == 0, TRIDA_ERR_ALIGN,
              "gdn_prep: conv_bias must be 16-byte aligned");
  TRIDA_CHECK(B * T < INT32_MAX, TRIDA_ERR_ARG, "gdn_prep: too many rows");
  PrepArgs a{x, window, conv_w, a_in, b_in, A_log, dt_bias, q, k, v, g, beta, window_out, pre_out,
             conv_bias, win_idx, pre_idx, cu_seqlens,
             (int)T, (int)C, (int)Kc, (int)Hk, (int)Hv, (int)Dk, (int)Dv, x_sb, x_st, ab_sb, ab_st};
  hipStream_t st = static_cast<hipStream_t>(stream);
  // small grids: 128-piece slices, one per block; grids of >= 512 rows (which fill the GPU anyway): one
  // block of 256 threads per row, up to 4 passes over its pieces, every pass's loads in flight together.
  // The passes are a template argument: each holds its loads in registers (4 x 16-byte source pieces,
  // 4 of weights, 1 of bias per thread), so a kernel built for more passes than the row needs would hold
  // registers for nothing and fit fewer blocks per CU
  const bool wide = B * T >= 512;
  TRIDA_CHECK(!wide || C <= 8 * 256 * 4, TRIDA_ERR_ARG, "gdn_prep: conv_dim %lld above %d", (long long)C, 8 * 256 * 4);
  const dim3 grid((unsigned)(B * T), wide ? 1u : (unsigned)cdiv(C / 8, 128));
  const bool idx = cu_seqlens || win_idx || pre_idx;
#define TRIDA_PREP_KC2(GW, NT, PS, IX)                                                                     \
  switch (Kc) {                                                                                            \
    case 2: hipLaunchKernelGGL((gdn_prep_kernel<GW, 2, NT, PS, IX>), grid, dim3(NT), 0, st, a); break;     \
    case 3: hipLaunchKernelGGL((gdn_prep_kernel<GW, 3, NT, PS, IX>), grid, dim3(NT), 0, st, a); break;     \
    default: hipLaunchKernelGGL((gdn_prep_kernel<GW, 4, NT, PS, IX>), grid, dim3(NT), 0, st, a); break;    \
  }
#define TRIDA_PREP_KC(GW, NT, PS)        \
  if (idx) {                             \
    TRIDA_PREP_KC2(GW, NT, PS, true)     \
  } else {                               \
    TRIDA_PREP_KC2(GW, NT, PS, false)    \
  }
  const int64_t passes = wide ? cdiv(C / 8, 256) : 1;
#define TRIDA_PREP_LAUNCH(GW)          \
  if (!wide) {                         \
    TRIDA_PREP_KC(GW, 128, 1)          \
  } else if (passes <= 1) {            \
    TRIDA_PREP_KC(GW, 256, 1)          \
  } else if (passes == 2) {            \
    TRIDA_PREP_KC(GW, 256, 2)          \
  } else if (passes == 3) {            \
    TRIDA_PREP_KC(GW, 256, 3)          \
  } else {                             \
    TRIDA_PREP_KC(GW, 256, 4)          \
  }
  switch (Dk) {
    case 32: TRIDA_PREP_LAUNCH(4) break;
    case 64: TRIDA_PREP_LAUNCH(8) break;
    default: TRIDA_PREP_LAUNCH(16) break;
  }
#undef TRIDA_PREP_LAUNCH
#undef TRIDA_PREP_KC
#undef TRIDA_PREP_KC2
  return launch_status("gdn_prep");
}
