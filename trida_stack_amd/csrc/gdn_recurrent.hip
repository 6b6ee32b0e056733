// Gated delta rule, token-recurrent form, with the block-causal canvas readout.
//
// Per value head h and row t (g = log decay, scale applied to q):
//   S = e^{g_t} S;  kv = S k_t;  delta = beta_t (v_t - kv);  S += delta k_t^T;  o_t = S q_t
// causal_mode 1: every row reads its own state. causal_mode 2: rows t < num_clean read their own
// state, rows t >= num_clean read the block-end state (the state after all T rows).
// Block-bidirectional readout (trida_gdr_block_bidir): per block of `bidir` rows, a backward sub-scan
// over the block's rows in reverse from the block-entry state, then the causal forward sub-scan; each
// row reads out the mean of the two; the state carried on is the forward one.
//
// Fused layer (trida_gdn_fused_layer, blocks of <= 64 rows): the block first runs the layer's front
// half itself -- depthwise causal conv over [window ++ x] + SiLU, l2norm of its q / k head, the gates
// g and beta -- from the pre-conv rows, staging the head's source rows in LDS, with the arithmetic of
// trida_gdn_prep in the same order (so the results are bit-identical to the two-kernel path). It
// writes the rows a rollback needs (k, v, g, beta, raw pre-conv rows, new window) only when asked.
//
// Launch: block = (sequence b, value head h, v-tile). Each wave owns 4 value columns; the 16 lanes of
// a column each hold KPL = Dk/16 consecutive k entries of that column's state in registers, so the
// two dot products of a step reduce over one 16-lane DPP row (no LDS round trip). The rows of q, k,
// v, g, beta are staged through LDS 32 at a time (all loads of a chunk in flight together).
// Critical path per step: decay, two independent dots (S'k and S'q), two interleaved row reductions,
// then o = S'q + delta (k.q); the state update itself is off the path.
//
// Gated-norm outputs (trida_gdr_recurrent_gnorm, small grids, one staged chunk): besides o, the block
// writes u = bf16(bf16(o) * w * silu(z)) of its value columns in the weight-streaming GEMM's fragment order
// and the sum of bf16(o)^2 over each 8 of its columns. The layer's gated RMSNorm, bf16(o * inv) * w * silu(z)
// with inv = rsqrt(mean_head(o^2) + eps), is then inv times u up to the rounding order: the out projection
// applies inv per row and head to its partial sums (trida_wsgemm_headnorm), so no kernel runs between the two.
#include "common.h"

namespace trida {
namespace {

constexpr int kLanesPerV = 16;
constexpr int kVPerWave = kWave / kLanesPerV;  // 4
constexpr int kTC = 64;                        // rows staged per LDS chunk (a canvas block fits in one)
constexpr int kTCF32 = 40;                     // the same, fp32-stage form

// A DPP lane permutation within 16-lane rows (row_ror and quad_perm read lanes of the same row only).
// Written as update_dpp with a defined old value and bound_ctrl so that the compiler folds it into the
// consuming add (v_add_f32 with a DPP source: one instruction instead of a mov and an add).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0x128>(v);  // row_ror:8
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  return v;
}
// Four independent 16-lane row sums, interleaved so the DPP latencies overlap.
__device__ __forceinline__ void row16_sum4(float (&v)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp<0x128>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp<0x124>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp<0x4E>(v[j]);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] += dpp<0xB1>(v[j]);
}
__device__ __forceinline__ void row16_sum2(float& a, float& b) {
  a += dpp<0x128>(a);
  b += dpp<0x128>(b);
  a += dpp<0x124>(a);
  b += dpp<0x124>(b);
  a += dpp<0x4E>(a);
  b += dpp<0x4E>(b);
  a += dpp<0xB1>(a);
  b += dpp<0xB1>(b);
}

constexpr int kMaxKc = 4;

// the fused layer's front half
struct PrepIn {
  const uint16_t* x;       // [B, T, C] pre-conv rows (batch stride x_sb, row stride x_st)
  const uint16_t* window;  // [B, Kc-1, C]
  const uint16_t* conv_w;  // [C, Kc]
  const uint16_t* a_in;    // [B, T, Hv] (batch stride ab_sb, row stride ab_st)
  const uint16_t* b_in;
  const float* A_log;  // [Hv]
  const float* dt_bias;
  uint16_t* k_out;  // [B, T, Hk, Dk] or null (rows kept for a rollback)
  uint16_t* v_out;  // [B, T, Hv, Dv] or null
  float* g_out;     // [B, T, Hv] or null (log decay)
  float* beta_out;
  uint16_t* pre_out;     // [slots, T, C] raw pre-conv rows or null
  uint16_t* window_out;  // [rows, Kc-1, C] new window or null
  const uint16_t* conv_bias;  // [C] or null
  const int32_t* win_idx;     // [B] window / window_out row of sequence b, or null (row b)
  const int32_t* pre_idx;     // [B] pre_out slot of sequence b, or null (slot b)
  int64_t x_sb, x_st, ab_sb, ab_st;
  int Kc;
};

struct RecArgs {
  const uint16_t* q;  // [B, T, Hk, Dk]
  const uint16_t* k;
  const uint16_t* v;  // [B, T, Hv, Dv]
  const float* g;     // [B, T, Hv]
  const float* beta;
  const float* state_in;  // [B, Hv, Dv, Dk]
  uint16_t* out;          // [B, T, Hv, Dv]
  float* state_out;
  float* state_clean;
  int T, Hk, Hv, Dk, Dv;
  int causal_mode, num_clean;
  float scale;
  int bidir;  // > 0: block-bidirectional readout over blocks of this many rows (causal_mode 1)
  PrepIn p;   // fused layer only
  const int32_t* cu_seqlens;  // [B + 1] packed ragged rows, or null (B x T rows)
  const int32_t* state_idx;   // [B] state_in / state_out row of sequence b, or null (row b)
  float* inter;               // [rows, csteps, Hv, Dv, Dk] states after rows 0..csteps-1, or null
  const int32_t* inter_idx;   // [B] inter row of sequence b, or null (row b)
  int csteps;
  // gated-norm outputs (F32 form, T <= one chunk): z rows (row stride gz_st), the norm weight [Dv], u in
  // fragment order [rows][Hv * Dv] and the partial sums of squares [rows][Hv][Dv / 8]; or null
  const uint16_t* gz;
  int64_t gz_st;
  const uint16_t* gw;
  uint16_t* gu;
  float* gss;
};

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

typedef __attribute__((address_space(3))) void lds_void;
// Copies n items of SZ bytes (4 or 16) to LDS, item i at dst + i * SZ, from the global address src(i),
// with direct-to-LDS loads: every load of the block stays in flight at once and no register holds the
// data. The caller waits for vmcnt(0), then a barrier, before reading dst.
template <int SZ, typename F>
__device__ __forceinline__ void lds_gather(void* dst, int n, F&& src, int nthreads) {
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave), lane = (int)threadIdx.x % kWave;
  for (int base = wave * kWave; base < n; base += nthreads)  // base is uniform over the wave
    if (base + lane < n)
      __builtin_amdgcn_global_load_lds(src(base + lane), (lds_void*)(static_cast<char*>(dst) + base * SZ), SZ, 0, 0);
}
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// F32 (small grids, no block-bidirectional readout): each staged chunk's k and q * scale are converted
// to fp32 once per block, so a row step reads them ready (the bf16 unpack and the scale multiply leave
// the per-step chain: 24 of ~80 instructions per step); chunks of 40 rows keep the fp32 stages within
// two blocks per CU. Large grids keep the bf16 stages, whose smaller LDS footprint holds more blocks.
// IDX: the pool / packed forms (cu_seqlens, state and window slot indices, the intermediate-state ring) may be in
// use; without it those pointers are ignored (null) and the plain form compiles without their loads and branches.
template <int KPL, int NW, bool PREP, bool F32, bool IDX>
__global__ __launch_bounds__(NW* kWave) void gdr_recurrent_kernel(RecArgs a) {
  const int32_t* cu_seqlens = IDX ? a.cu_seqlens : nullptr;
  const int32_t* state_idx = IDX ? a.state_idx : nullptr;
  float* inter = IDX ? a.inter : nullptr;
  const int32_t* inter_idx = IDX ? a.inter_idx : nullptr;
  constexpr int TC = F32 ? kTCF32 : kTC;  // rows staged per chunk
  constexpr int Dk = KPL * kLanesPerV;
  constexpr int VPB = NW * kVPerWave;
  const int tiles = a.Dv / VPB;
  const int bid = xcd_major(blockIdx.x, gridDim.x);  // a head's value tiles (same q / k rows) on one XCD
  const int vt = bid % tiles;
  const int h = (bid / tiles) % a.Hv;
  const int b = bid / (tiles * a.Hv);
  const int hk = h / (a.Hv / a.Hk);
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int vl = wave * kVPerWave + lane / kLanesPerV;  // value column within the tile
  const int v = vt * VPB + vl;
  const int kl = lane % kLanesPerV;                      // k slice [kl*KPL, kl*KPL+KPL)
  // the sequence's rows: [row0, row0 + T) of the packed arrays (B x a.T rows unless cu_seqlens is given)
  int64_t row0 = (int64_t)b * a.T;
  int T = a.T;
  if (cu_seqlens) {
    row0 = cu_seqlens[b];
    T = max(0, min(cu_seqlens[b + 1] - (int)row0, a.T));
  }

  __shared__ __align__(16) uint16_t s_q[TC][Dk];
  __shared__ __align__(16) uint16_t s_k[TC][Dk];
  __shared__ __align__(16) float s_qf32[F32 ? TC : 1][F32 ? Dk : 4];  // q * scale (F32 form)
  __shared__ __align__(16) float s_kf32[F32 ? TC : 1][F32 ? Dk : 4];  // k (F32 form)
  __shared__ __align__(16) uint16_t s_v[TC][VPB];
  __shared__ float s_g[TC], s_b[TC];
  __shared__ float s_ob[TC][VPB];  // backward sub-scan outputs of the block-bidirectional readout
  __shared__ float s_kq[TC];  // k . (q * scale) per staged row
  // entry i of staged row r: k, and q * scale (the same product on both forms)
  auto kval = [&](int r, int i) -> float {
    if constexpr (F32) return s_kf32[r][i];
    else return bf2f(s_k[r][i]);
  };
  auto qval = [&](int r, int i) -> float {
    if constexpr (F32) return s_qf32[r][i];
    else return bf2f(s_q[r][i]) * a.scale;
  };

  const int64_t col_off = ((int64_t)h * a.Dv + v) * Dk + kl * KPL;  // within one [Hv, Dv, Dk] state
  // gated-norm outputs: thread e < T * VPB / 8 owns row e / (VPB / 8), 8 columns; its z and w pieces load
  // with the first memory round trip
  constexpr int GPR = VPB / 8 > 0 ? VPB / 8 : 1;  // 8-column pieces of a row of the tile
  u32x4 gzr = u32x4{0u, 0u, 0u, 0u}, gwr = u32x4{0u, 0u, 0u, 0u};
  const bool gown = F32 && a.gu && tid < T * GPR;
  if (gown) {
    const int gc = h * a.Dv + vt * VPB + (tid % GPR) * 8;  // first column within the z row / u row
    gzr = *reinterpret_cast<const u32x4*>(a.gz + (row0 + tid / GPR) * a.gz_st + gc);
    gwr = *reinterpret_cast<const u32x4*>(a.gw + vt * VPB + (tid % GPR) * 8);
  }
  const int64_t hvk = (int64_t)a.Hv * a.Dv * Dk;
  const int64_t st_off = (state_idx ? state_idx[b] : b) * hvk + col_off;  // state_in / state_out
  const int64_t cl_off = (int64_t)b * hvk + col_off;                           // state_clean
  float s[KPL];
#pragma unroll
  for (int i = 0; i < KPL; ++i) s[i] = a.state_in[st_off + i];
  // the intermediate states: after row t, t < csteps, of this sequence
  const int csteps = inter ? min(a.csteps, T) : 0;
  float* inter_col = inter ? inter + (int64_t)(inter_idx ? inter_idx[b] : b) * a.csteps * hvk + col_off : nullptr;

  const int nc = a.causal_mode == 2 ? min(a.num_clean, T) : T;
  const int64_t qk_row = (int64_t)a.Hk * Dk;  // elements between rows t and t+1
  const uint16_t* qb = a.q + row0 * qk_row + (int64_t)hk * Dk;
  const uint16_t* kb = a.k + row0 * qk_row + (int64_t)hk * Dk;
  const int64_t v_row = (int64_t)a.Hv * a.Dv;
  const uint16_t* vb = a.v + row0 * v_row + (int64_t)h * a.Dv + vt * VPB;
  uint16_t* ob = a.out + row0 * v_row + (int64_t)h * a.Dv + v;
  const float* gb = a.g + row0 * a.Hv + h;
  const float* bb = a.beta + row0 * a.Hv + h;

  // rows staged per chunk: whole blocks when the readout is block-bidirectional
  const int tcn = a.bidir > 0 ? (TC / a.bidir) * a.bidir : TC;
  // one step of the recurrence on state st with staged row r; returns the row's readout S'q
  auto step = [&](float (&st)[KPL], int r) -> float {
    float kk[KPL], qq[KPL];
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      kk[i] = kval(r, kl * KPL + i);
      qq[i] = qval(r, kl * KPL + i);
    }
    const float eg = s_g[r];
    float kv = 0.f, sq = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      st[i] *= eg;
      kv = fmaf(st[i], kk[i], kv);
      sq = fmaf(st[i], qq[i], sq);
    }
    row16_sum2(kv, sq);
    const float delta = (bf2f(s_v[r][vl]) - kv) * s_b[r];
#pragma unroll
    for (int i = 0; i < KPL; ++i) st[i] = fmaf(kk[i], delta, st[i]);
    return fmaf(delta, s_kq[r], sq);
  };
  if constexpr (PREP) {
    // ---- front half: conv + SiLU + l2norm + gates for this block's head, all T (<= kTC) rows ----
    constexpr int NT = NW * kWave;
    constexpr int GW = Dk / 8;    // 8-channel pieces per q or k head
    constexpr int QKP = 2 * GW;   // q pieces then k pieces
    __shared__ __align__(16) uint16_t s_src[kTC + kMaxKc - 1][2 * Dk];  // [window ++ x] rows, q|k channels
    __shared__ __align__(16) uint16_t s_vsrc[kTC + kMaxKc - 1][VPB];
    __shared__ __align__(16) uint16_t s_qkw[2][Dk * kMaxKc];  // conv weights [channel][tap], q then k head
    __shared__ __align__(16) uint16_t s_vw[VPB * kMaxKc];
    const PrepIn& p = a.p;
    const int Kc = p.Kc, W = Kc - 1, nsrc = T + W;
    const int key_dim = a.Hk * Dk, C = 2 * key_dim + a.Hv * a.Dv;
    const uint16_t* xs = p.x + (int64_t)b * p.x_sb;
    const int wrow = (IDX && p.win_idx) ? p.win_idx[b] : b;
    const int pslot = (IDX && p.pre_idx) ? p.pre_idx[b] : b;
    const uint16_t* ws = p.window + (int64_t)wrow * W * C;
    auto src_row = [&](int i) { return i < W ? ws + (int64_t)i * C : xs + (int64_t)(i - W) * p.x_st; };
    auto qk_chan = [&](int pc) { return (pc < GW ? hk * Dk : key_dim + hk * Dk - GW * 8) + pc * 8; };
    const int vc0 = 2 * key_dim + h * a.Dv + vt * VPB;  // this block's first v channel
    // every input of the front half in one round trip: rows and weights straight to LDS, the gate
    // inputs into registers (T <= kTC <= NT: one row per thread)
    lds_gather<16>(&s_src[0][0], nsrc * QKP, [&](int i) { return (const void*)(src_row(i / QKP) + qk_chan(i % QKP)); }, NT);
    lds_gather<4>(&s_vsrc[0][0], nsrc * (VPB / 2),
                  [&](int i) { return (const void*)(src_row(i / (VPB / 2)) + vc0 + (i % (VPB / 2)) * 2); }, NT);
    lds_gather<16>(&s_qkw[0][0], Dk * Kc / 8, [&](int i) { return (const void*)(p.conv_w + (int64_t)hk * Dk * Kc + i * 8); }, NT);
    lds_gather<16>(&s_qkw[1][0], Dk * Kc / 8,
                   [&](int i) { return (const void*)(p.conv_w + (int64_t)(key_dim + hk * Dk) * Kc + i * 8); }, NT);
    lds_gather<4>(&s_vw[0], VPB * Kc / 2, [&](int i) { return (const void*)(p.conv_w + (int64_t)vc0 * Kc + i * 2); }, NT);
    const bool grow = tid < T;
    float av = 0.f, bv = 0.f;
    if (grow) {
      av = bf2f(p.a_in[(int64_t)b * p.ab_sb + (int64_t)tid * p.ab_st + h]);
      bv = bf2f(p.b_in[(int64_t)b * p.ab_sb + (int64_t)tid * p.ab_st + h]);
    }
    const float alog = p.A_log[h], dtb = p.dt_bias[h];
    wait_vmem();
    // one block per q/k head (and per value head for g, beta) writes the shared rows
    const bool qk_writer = vt == 0 && h % (a.Hv / a.Hk) == 0;
    if (grow) {
      const float gl = -__expf(alog) * softplus(av + dtb);
      const float be = 1.f / (1.f + __expf(-bv));
      s_g[tid] = __expf(gl);
      s_b[tid] = be;
      if (vt == 0 && p.g_out) {
        const int64_t o = (row0 + tid) * a.Hv + h;
        p.g_out[o] = gl;
        p.beta_out[o] = be;
      }
    }
    __syncthreads();
    // q / k: a thread owns one piece; the GW lanes of a head reduce its sum of squares together, so
    // every lane of a group walks the same rows (rows past T are computed and dropped)
    {
      const int pc = tid % QKP, part = tid / QKP, nparts = NT / QKP;
      float w[8][kMaxKc];
#pragma unroll
      for (int ch = 0; ch < 8; ++ch)
#pragma unroll
        for (int j = 0; j < kMaxKc; ++j)
          w[ch][j] = j < Kc ? bf2f(s_qkw[pc < GW ? 0 : 1][((pc % GW) * 8 + ch) * Kc + j]) : 0.f;
      const int tpad = (T + nparts - 1) / nparts * nparts;
      float bias[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (p.conv_bias) unpack8(*reinterpret_cast<const u32x4*>(p.conv_bias + qk_chan(pc)), bias);
      for (int t = part; t < tpad; t += nparts) {
        float acc[8];
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) acc[ch] = bias[ch];
#pragma unroll
        for (int j = 0; j < kMaxKc; ++j) {
          if (j < Kc) {
            float f[8];
            unpack8(*reinterpret_cast<const u32x4*>(&s_src[t + j][pc * 8]), f);
#pragma unroll
            for (int ch = 0; ch < 8; ++ch) acc[ch] = fmaf(w[ch][j], f[ch], acc[ch]);
          }
        }
        float ss = 0.f;
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) {
          acc[ch] = bf2f(f2bf(silu(acc[ch])));
          ss = fmaf(acc[ch], acc[ch], ss);
        }
        ss = lane_group_sum<GW>(ss);
        const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) acc[ch] *= inv;
        if (t < T) {
          const u32x4 pk = pack8(acc);
          if (pc < GW) {
            *reinterpret_cast<u32x4*>(&s_q[t][pc * 8]) = pk;
          } else {
            *reinterpret_cast<u32x4*>(&s_k[t][(pc - GW) * 8]) = pk;
            if (qk_writer && p.k_out)
              *reinterpret_cast<u32x4*>(p.k_out + ((row0 + t) * a.Hk + hk) * Dk + (pc - GW) * 8) = pk;
          }
        }
      }
    }
    // v: one (row, column) per thread
    for (int e = tid; e < T * VPB; e += NT) {
      const int t = e / VPB, cc = e % VPB;
      float acc = p.conv_bias ? bf2f(p.conv_bias[vc0 + cc]) : 0.f;
      for (int j = 0; j < Kc; ++j) acc = fmaf(bf2f(s_vw[cc * Kc + j]), bf2f(s_vsrc[t + j][cc]), acc);
      const uint16_t vb16 = f2bf(silu(acc));
      s_v[t][cc] = vb16;
      if (p.v_out) p.v_out[(row0 + t) * a.Hv * a.Dv + h * a.Dv + vt * VPB + cc] = vb16;
    }
    // raw pre-conv rows and the new window (last Kc-1 rows of [window ++ x]) of this block's channels
    if (p.pre_out || p.window_out) {
      for (int e = tid; e < nsrc * QKP; e += NT) {
        const int i = e / QKP, pc = e % QKP;
        if (!qk_writer) break;
        const u32x4 val = *reinterpret_cast<const u32x4*>(&s_src[i][pc * 8]);
        if (p.pre_out && i >= W)
          *reinterpret_cast<u32x4*>(p.pre_out + ((int64_t)pslot * T + (i - W)) * C + qk_chan(pc)) = val;
        if (p.window_out && i >= nsrc - W)
          *reinterpret_cast<u32x4*>(p.window_out + ((int64_t)wrow * W + (i - (nsrc - W))) * C + qk_chan(pc)) = val;
      }
      for (int e = tid; e < nsrc * VPB; e += NT) {
        const int i = e / VPB, cc = e % VPB;
        const uint16_t val = s_vsrc[i][cc];
        if (p.pre_out && i >= W) p.pre_out[((int64_t)pslot * T + (i - W)) * C + vc0 + cc] = val;
        if (p.window_out && i >= nsrc - W) p.window_out[((int64_t)wrow * W + (i - (nsrc - W))) * C + vc0 + cc] = val;
      }
    }
    __syncthreads();
  }
  // a row's operands in registers, and the step on them (the same arithmetic as step())
  struct Row {
    float kk[KPL], qq[KPL];
    float eg, vv, be, kq;
  };
  auto fetch = [&](Row& R, int r) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      R.kk[i] = kval(r, kl * KPL + i);
      R.qq[i] = qval(r, kl * KPL + i);
    }
    R.eg = s_g[r];
    R.vv = bf2f(s_v[r][vl]);
    R.be = s_b[r];
    R.kq = s_kq[r];
  };
  auto apply = [&](float (&st)[KPL], const Row& R) -> float {
    float kv = 0.f, sq = 0.f;
#pragma unroll
    for (int i = 0; i < KPL; ++i) {
      st[i] *= R.eg;
      kv = fmaf(st[i], R.kk[i], kv);
      sq = fmaf(st[i], R.qq[i], sq);
    }
    row16_sum2(kv, sq);
    const float delta = (R.vv - kv) * R.be;
#pragma unroll
    for (int i = 0; i < KPL; ++i) st[i] = fmaf(R.kk[i], delta, st[i]);
    return fmaf(delta, R.kq, sq);
  };
  for (int t0 = 0; t0 < T; t0 += tcn) {
    const int tn = min(tcn, T - t0);
    if constexpr (F32) {
      __syncthreads();  // previous chunk fully consumed (its readout rows stored)
      // stage the chunk through registers in one round trip (clamped, unconditional loads): q * scale and
      // k converted to fp32 once, the v tile, g and beta; with KPL = 8 the thread holding piece j of a row
      // also forms lane j's share of k . (q * scale) -- the slice and fma order of the separate pass below
      // -- and its 16-lane group (the row's 16 pieces) reduces it with the same row16_sum
      constexpr int NT = NW * kWave;
      constexpr int PPR = Dk / 8;  // 16-byte pieces per q / k row
      constexpr int QIT = (TC * PPR + NT - 1) / NT;
      constexpr int VW = VPB / 2;  // 4-byte pieces per v tile row
      constexpr int VIT = (TC * VW + NT - 1) / NT;
      const int nq = tn * PPR, nv = tn * VW;
      const uint16_t* qc = qb + (int64_t)t0 * qk_row;
      const uint16_t* kc = kb + (int64_t)t0 * qk_row;
      const uint16_t* vc = vb + (int64_t)t0 * v_row;
      u32x4 qr[QIT], kr[QIT];
      uint32_t vr[VIT];
#pragma unroll
      for (int it = 0; it < QIT; ++it) {
        const int i = min(tid + it * NT, nq - 1);
        const int off = (i / PPR) * (int)qk_row + (i % PPR) * 8;
        qr[it] = *reinterpret_cast<const u32x4*>(qc + off);
        kr[it] = *reinterpret_cast<const u32x4*>(kc + off);
      }
#pragma unroll
      for (int it = 0; it < VIT; ++it) {
        const int i = min(tid + it * NT, nv - 1);
        vr[it] = *reinterpret_cast<const uint32_t*>(vc + (i / VW) * (int)v_row + (i % VW) * 2);
      }
      const int tr = min(tid, tn - 1);
      const float gv = gb[(int64_t)(t0 + tr) * a.Hv], bv = bb[(int64_t)(t0 + tr) * a.Hv];
      if (tid < tn) {
        s_g[tid] = __expf(gv);
        s_b[tid] = bv;
      }
#pragma unroll
      for (int it = 0; it < VIT; ++it) {
        const int i = tid + it * NT;
        if (i < nv) *reinterpret_cast<uint32_t*>(&s_v[i / VW][(i % VW) * 2]) = vr[it];
      }
#pragma unroll
      for (int it = 0; it < QIT; ++it) {
        const int i = tid + it * NT;
        if (i < nq) {  // whole rows: uniform over each 16-lane group
          const int row = i / PPR, pc = i % PPR;
          float qf[8], kf[8];
          unpack8(qr[it], qf);
          unpack8(kr[it], kf);
          float kq = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            qf[j] *= a.scale;
            kq = fmaf(kf[j], qf[j], kq);
          }
          *reinterpret_cast<f32x4*>(&s_qf32[row][pc * 8]) = f32x4{qf[0], qf[1], qf[2], qf[3]};
          *reinterpret_cast<f32x4*>(&s_qf32[row][pc * 8 + 4]) = f32x4{qf[4], qf[5], qf[6], qf[7]};
          *reinterpret_cast<f32x4*>(&s_kf32[row][pc * 8]) = f32x4{kf[0], kf[1], kf[2], kf[3]};
          *reinterpret_cast<f32x4*>(&s_kf32[row][pc * 8 + 4]) = f32x4{kf[4], kf[5], kf[6], kf[7]};
          if constexpr (KPL == 8) {
            kq = row16_sum(kq);
            if (pc == 0) s_kq[row] = kq;
          }
        }
      }
      __syncthreads();
    } else if constexpr (!PREP) {
    __syncthreads();  // previous chunk fully consumed
    // stage q, k rows (16-byte pieces) and the v tile straight to LDS, g and beta through registers
    // (tn <= kTC <= block size: one row per thread), all in one round trip
    constexpr int kPieces = Dk / 8;
    lds_gather<16>(&s_q[0][0], tn * kPieces,
                   [&](int i) { return (const void*)(qb + (int64_t)(t0 + i / kPieces) * qk_row + (i % kPieces) * 8); },
                   NW * kWave);
    lds_gather<16>(&s_k[0][0], tn * kPieces,
                   [&](int i) { return (const void*)(kb + (int64_t)(t0 + i / kPieces) * qk_row + (i % kPieces) * 8); },
                   NW * kWave);
    lds_gather<4>(&s_v[0][0], tn * (VPB / 2),
                  [&](int i) { return (const void*)(vb + (int64_t)(t0 + i / (VPB / 2)) * v_row + (i % (VPB / 2)) * 2); },
                  NW * kWave);
    float gv = 0.f, bv = 0.f;
    if (tid < tn) {
      gv = gb[(int64_t)(t0 + tid) * a.Hv];
      bv = bb[(int64_t)(t0 + tid) * a.Hv];
    }
    wait_vmem();
    if (tid < tn) {
      s_g[tid] = __expf(gv);
      s_b[tid] = bv;
    }
    __syncthreads();
    }
    if constexpr (!F32 || KPL != 8) {
      // k . (q * scale) of every staged row, once per block instead of once per value column: each
      // 16-lane group takes a row, lane j the same KPL-element slice and fma order as the column lanes'
      // row step, then the same row16_sum, so the value is the one a row step would compute itself
      for (int rr = tid / kLanesPerV; rr < tn; rr += NW * kVPerWave) {  // uniform within a 16-lane group
        const int j = tid % kLanesPerV;
        float kq = 0.f;
#pragma unroll
        for (int i = 0; i < KPL; ++i)
          kq = fmaf(kval(rr, j * KPL + i), qval(rr, j * KPL + i), kq);
        kq = row16_sum(kq);
        if (j == 0) s_kq[rr] = kq;
      }
      __syncthreads();
    }
    if (a.bidir > 0) {
      // each block: a backward sub-scan from the block-entry state (a register copy), then the causal
      // forward sub-scan; a row reads out the mean of the two
      for (int r0 = 0; r0 < tn; r0 += a.bidir) {
        const int r1 = min(r0 + a.bidir, tn);
        float sb[KPL];
#pragma unroll
        for (int i = 0; i < KPL; ++i) sb[i] = s[i];
        for (int r = r1 - 1; r >= r0; --r) {
          const float o = step(sb, r);
          if (kl == 0) s_ob[r][vl] = o;
        }
        for (int r = r0; r < r1; ++r) {
          const float o = step(s, r);
          if (kl == 0) ob[(int64_t)(t0 + r) * v_row] = f2bf(0.5f * (o + s_ob[r][vl]));
        }
      }
      continue;
    }
    // rows [r0, r1) of the chunk; the next row's operands are read from LDS while the current row computes
    // (two register sets, unconditional reads of a clamped row, so the waits are the same on every path).
    // A row's readout: F32 keeps it in LDS (every lane of a column holds the same reduced value) and the
    // block stores the chunk's rows together; otherwise lane 0 of the column stores it
    auto run = [&](int r0, int r1, bool keep) {
      if (r0 >= r1) return;
      auto put = [&](int r, float o) {
        if constexpr (F32) {
          if (keep) s_ob[r][vl] = o;
        } else {
          if (keep && kl == 0) ob[(int64_t)(t0 + r) * v_row] = f2bf(o);
        }
      };
      // the state after row r, when the caller keeps intermediates (uniform branch)
      auto stash = [&](int r) {
        if (IDX && t0 + r < csteps) {
#pragma unroll
          for (int i = 0; i < KPL; ++i) inter_col[(int64_t)(t0 + r) * hvk + i] = s[i];
        }
      };
      Row ra, rb;
      fetch(ra, r0);
      int r = r0;
      for (; r + 1 < r1; r += 2) {
        fetch(rb, r + 1);
        put(r, apply(s, ra));
        stash(r);
        fetch(ra, min(r + 2, r1 - 1));
        put(r + 1, apply(s, rb));
        stash(r + 1);
      }
      if (r < r1) {
        put(r, apply(s, ra));
        stash(r);
      }
    };
    const int rc = min(max(nc - t0, 0), tn);  // the chunk's rows t < nc, whose readout is kept
    run(0, rc, true);
    if (a.state_clean && rc > 0 && t0 + rc == nc) {  // the state after the last clean row
#pragma unroll
      for (int i = 0; i < KPL; ++i) a.state_clean[cl_off + i] = s[i];
    }
    run(rc, tn, false);
    if constexpr (F32) {
      __syncthreads();
      uint16_t* otile = a.out + row0 * v_row + (int64_t)h * a.Dv + vt * VPB;
      for (int e = tid; e < rc * VPB; e += NW * kWave)
        otile[(int64_t)(t0 + e / VPB) * v_row + e % VPB] = f2bf(s_ob[e / VPB][e % VPB]);
    }
  }
  if (nc == 0 && a.state_clean) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) a.state_clean[cl_off + i] = a.state_in[st_off + i];
  }
  // MASK rows (causal_mode 2): read the block-end state, four rows at a time. On a large grid (many
  // sequences: issue-bound) their q * scale is formed once per block in fp32 (the same products the
  // per-lane path forms) into the k stage, dead after the causal rows: its kTC x Dk bf16 hold kTC / 2
  // rows of Dk fp32 (batch 64: 184 -> 170 us per layer). On a grid of a few hundred blocks (batch 1:
  // latency-bound) the two barriers cost more than they save, so each lane converts its own q.
  const int nm = T - nc;
  const bool qf_staged = !F32 && (PREP || T <= tcn) && nm > 0 && nm <= TC / 2 && gridDim.x >= 1024;  // block-uniform
  float* s_qf = reinterpret_cast<float*>(&s_k[0][0]);
  if (qf_staged) {
    __syncthreads();  // every wave is done with the k rows
    for (int e = tid; e < nm * Dk; e += NW * kWave) s_qf[e] = bf2f(s_q[nc + e / Dk][e % Dk]) * a.scale;
    __syncthreads();
  }
  if (F32 && T <= tcn && nm > 0) {
    // the whole block is the last staged chunk (s_qf32 holds every row): eight rows at a time, two
    // interleaved 4-row reductions (each row's fma order and row16 reduction as below), the readouts
    // kept in LDS and stored together
    for (int t = nc; t < T; t += 8) {
      float o0[4], o1[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ta = min(t + j, T - 1), tb = min(t + 4 + j, T - 1);
        o0[j] = 0.f;
        o1[j] = 0.f;
#pragma unroll
        for (int i = 0; i < KPL; ++i) {
          o0[j] = fmaf(s[i], s_qf32[ta][kl * KPL + i], o0[j]);
          o1[j] = fmaf(s[i], s_qf32[tb][kl * KPL + i], o1[j]);
        }
      }
      row16_sum4(o0);
      row16_sum4(o1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (t + j < T) s_ob[t + j][vl] = o0[j];
        if (t + 4 + j < T) s_ob[t + 4 + j][vl] = o1[j];
      }
    }
    __syncthreads();
    uint16_t* otile = a.out + row0 * v_row + (int64_t)h * a.Dv + vt * VPB;
    for (int e = tid; e < nm * VPB; e += NW * kWave)
      otile[(int64_t)(nc + e / VPB) * v_row + e % VPB] = f2bf(s_ob[nc + e / VPB][e % VPB]);
  } else
  for (int t = nc; t < T; t += 4) {
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int tt = min(t + j, T - 1);
      o[j] = 0.f;
      if (F32 && T <= tcn) {  // the whole block is the last staged chunk
#pragma unroll
        for (int i = 0; i < KPL; ++i) o[j] = fmaf(s[i], s_qf32[tt][kl * KPL + i], o[j]);
      } else if (qf_staged) {
        const float* qr = s_qf + (tt - nc) * Dk + kl * KPL;
#pragma unroll
        for (int i = 0; i < KPL; ++i) o[j] = fmaf(s[i], qr[i], o[j]);
      } else {
        // the lane's KPL entries of q row tt: from LDS when the whole block was staged
        const uint16_t* qr = ((PREP || T <= tcn) ? &s_q[tt][0] : qb + (int64_t)tt * qk_row) + kl * KPL;
#pragma unroll
        for (int i = 0; i < KPL; ++i) o[j] = fmaf(s[i], bf2f(qr[i]) * a.scale, o[j]);
      }
    }
    row16_sum4(o);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (t + j < T && kl == 0) ob[(int64_t)(t + j) * v_row] = f2bf(o[j]);
  }
  if (F32 && a.gu) {
    __syncthreads();  // every row's readout is in s_ob (T <= one chunk)
    if (gown) {
      const int t = tid / GPR, pc = tid % GPR;
      float zf[8], wf[8], u[8];
      unpack8(gzr, zf);
      unpack8(gwr, wf);
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float o = bf2f(f2bf(s_ob[t][pc * 8 + c]));  // the bf16 output the norm reads
        ss = fmaf(o, o, ss);
        u[c] = o * wf[c] * (zf[c] / (1.f + __expf(-zf[c])));
      }
      *reinterpret_cast<u32x4*>(a.gu + ws_frag_off((int)(row0 + t), (int64_t)h * a.Dv + vt * VPB + pc * 8)) = pack8(u);
      a.gss[((row0 + t) * a.Hv + h) * (a.Dv / 8) + vt * GPR + pc] = ss;
    }
  }
  if (a.state_out) {
#pragma unroll
    for (int i = 0; i < KPL; ++i) a.state_out[st_off + i] = s[i];
  }
}

template <int KPL, bool PREP, bool F32, bool IDX>
void launch_nw2(const RecArgs& a, int nw, unsigned grid, hipStream_t st) {
  switch (nw) {
    case 4: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 4, PREP, F32, IDX>), dim3(grid), dim3(4 * kWave), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 2, PREP, F32, IDX>), dim3(grid), dim3(2 * kWave), 0, st, a); break;
    default: hipLaunchKernelGGL((gdr_recurrent_kernel<KPL, 1, PREP, F32, IDX>), dim3(grid), dim3(kWave), 0, st, a); break;
  }
}
template <int KPL, bool PREP, bool F32>
void launch_nw(const RecArgs& a, int nw, unsigned grid, hipStream_t st) {
  if (a.cu_seqlens || a.state_idx || a.inter || a.inter_idx || a.p.win_idx || a.p.pre_idx)
    launch_nw2<KPL, PREP, F32, true>(a, nw, grid, st);
  else
    launch_nw2<KPL, PREP, F32, false>(a, nw, grid, st);
}

template <int KPL, bool PREP = false>
int launch_kpl(const RecArgs& a, int B, hipStream_t st) {
  // widest block whose v-tile divides Dv; more, narrower blocks when the grid would be small
  int nw = 4;
  const int nw_min = a.gu ? 2 : 1;  // the gated-norm outputs take whole 8-column pieces
  while (nw > nw_min && (a.Dv % (nw * kVPerWave) != 0 || (int64_t)B * a.Hv * (a.Dv / (nw * kVPerWave)) < 256)) nw /= 2;
  if (a.Dv % (nw * kVPerWave) != 0) return TRIDA_ERR_ARG;
  const unsigned grid = (unsigned)((int64_t)B * a.Hv * (a.Dv / (nw * kVPerWave)));
  // fp32 stages on grids of fewer than 1024 blocks (batch 1: 512), where a block's row chain is the
  // critical path and two blocks per CU already hold the grid
  const bool f32 = !PREP && a.bidir == 0 && grid < 1024;
  // the gated-norm outputs: the fp32-stage form with one chunk, whole 8-column pieces, one per thread
  if (a.gu && (!f32 || a.T > kTCF32 || (nw * kVPerWave) % 8 != 0 || a.T * (nw * kVPerWave / 8) > nw * kWave)) {
    set_error("gdr_recurrent_gnorm: needs a grid of < 1024 blocks and T <= %d (got T=%d, %u blocks)", kTCF32, a.T,
              grid);
    return TRIDA_ERR_ARG;
  }
  if (f32)
    launch_nw<KPL, PREP, !PREP>(a, nw, grid, st);
  else
    launch_nw<KPL, PREP, false>(a, nw, grid, st);
  return launch_status(PREP ? "gdn_fused_layer" : "gdr_recurrent");
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int trida_gdr_recurrent(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                   const float* beta, const float* state_in, uint16_t* out, float* state_out,
                                   float* state_clean, int64_t B, int64_t T, int64_t Hk, int64_t Hv,
                                   int64_t Dk, int64_t Dv, int causal_mode, int64_t num_clean, float scale,
                                   const int32_t* cu_seqlens, const int32_t* state_idx, float* inter,
                                   const int32_t* inter_idx, int64_t cache_steps, void* stream) {
  TRIDA_CHECK(q && k && v && g && beta && state_in && out, TRIDA_ERR_NULL,
              "gdr_recurrent: q, k, v, g, beta, state_in and out are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, TRIDA_ERR_ARG,
              "gdr_recurrent: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld", (long long)B, (long long)T,
              (long long)Hk, (long long)Hv);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128 || Dk == 256, TRIDA_ERR_ARG,
              "gdr_recurrent: Dk must be 32, 64, 128 or 256 (got %lld)", (long long)Dk);
  TRIDA_CHECK(Dv > 0 && Dv % 4 == 0, TRIDA_ERR_ARG, "gdr_recurrent: Dv must be a multiple of 4");
  TRIDA_CHECK(causal_mode == 1 || causal_mode == 2, TRIDA_ERR_ARG, "gdr_recurrent: causal_mode is 1 or 2");
  TRIDA_CHECK(num_clean >= 0, TRIDA_ERR_ARG, "gdr_recurrent: num_clean >= 0");
  TRIDA_CHECK(state_clean == nullptr || (state_clean != state_in && state_clean != state_out), TRIDA_ERR_ARG,
              "gdr_recurrent: state_clean must not alias state_in or state_out");
  TRIDA_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 3) == 0, TRIDA_ERR_ALIGN,
              "gdr_recurrent: q and k must be 16-byte aligned, v 4-byte aligned");
  TRIDA_CHECK(B * T * Hv < INT32_MAX, TRIDA_ERR_ARG, "gdr_recurrent: problem too large");
  TRIDA_CHECK(inter == nullptr || (cache_steps >= 1 && cache_steps <= INT32_MAX), TRIDA_ERR_ARG,
              "gdr_recurrent: cache_steps >= 1 with inter");
  TRIDA_CHECK(inter == nullptr || ((uintptr_t)inter & 15) == 0, TRIDA_ERR_ALIGN, "gdr_recurrent: inter 16-byte aligned");
  RecArgs a{q, k, v, g, beta, state_in, out, state_out, state_clean, (int)T, (int)Hk, (int)Hv, (int)Dk,
            (int)Dv, causal_mode, (int)num_clean, scale, 0, PrepIn{}, cu_seqlens, state_idx, inter, inter_idx,
            inter ? (int)cache_steps : 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2>(a, (int)B, st);
    case 64: return launch_kpl<4>(a, (int)B, st);
    case 128: return launch_kpl<8>(a, (int)B, st);
    default: return launch_kpl<16>(a, (int)B, st);
  }
}

extern "C" int trida_gdr_recurrent_gnorm(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                         const float* beta, const float* state_in, uint16_t* out, float* state_out,
                                         float* state_clean, int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk,
                                         int64_t Dv, int causal_mode, int64_t num_clean, float scale,
                                         const uint16_t* z, int64_t z_row_stride, const uint16_t* gnorm_w,
                                         uint16_t* u_frag, float* ss_parts, void* stream) {
  TRIDA_CHECK(q && k && v && g && beta && state_in && out && z && gnorm_w && u_frag && ss_parts, TRIDA_ERR_NULL,
              "gdr_recurrent_gnorm: q, k, v, g, beta, state_in, out, z, gnorm_w, u_frag and ss_parts are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0 && B * T <= 48, TRIDA_ERR_ARG,
              "gdr_recurrent_gnorm: bad sizes B=%lld T=%lld Hk=%lld Hv=%lld (B T <= 48)", (long long)B, (long long)T,
              (long long)Hk, (long long)Hv);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128 || Dk == 256, TRIDA_ERR_ARG,
              "gdr_recurrent_gnorm: Dk must be 32, 64, 128 or 256 (got %lld)", (long long)Dk);
  TRIDA_CHECK(Dv % 32 == 0, TRIDA_ERR_ARG, "gdr_recurrent_gnorm: Dv must be a multiple of 32");
  TRIDA_CHECK(causal_mode == 1 || causal_mode == 2, TRIDA_ERR_ARG, "gdr_recurrent_gnorm: causal_mode is 1 or 2");
  TRIDA_CHECK(num_clean >= 0, TRIDA_ERR_ARG, "gdr_recurrent_gnorm: num_clean >= 0");
  TRIDA_CHECK(state_clean == nullptr || (state_clean != state_in && state_clean != state_out), TRIDA_ERR_ARG,
              "gdr_recurrent_gnorm: state_clean must not alias state_in or state_out");
  TRIDA_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 3) == 0 &&
                  ((uintptr_t)z & 15) == 0 && z_row_stride % 8 == 0 && z_row_stride >= Hv * Dv &&
                  ((uintptr_t)gnorm_w & 15) == 0 && ((uintptr_t)u_frag & 15) == 0 && ((uintptr_t)ss_parts & 3) == 0,
              TRIDA_ERR_ALIGN, "gdr_recurrent_gnorm: q, k, z, gnorm_w and u_frag 16-byte aligned (z rows of >= Hv Dv "
              "elements, a multiple of 8), v and ss_parts 4-byte aligned");
  RecArgs a{q, k, v, g, beta, state_in, out, state_out, state_clean, (int)T, (int)Hk, (int)Hv, (int)Dk,
            (int)Dv, causal_mode, (int)num_clean, scale, 0, PrepIn{}, nullptr, nullptr, nullptr, nullptr, 0,
            z, z_row_stride, gnorm_w, u_frag, ss_parts};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2>(a, (int)B, st);
    case 64: return launch_kpl<4>(a, (int)B, st);
    case 128: return launch_kpl<8>(a, (int)B, st);
    default: return launch_kpl<16>(a, (int)B, st);
  }
}

extern "C" int trida_gdr_block_bidir(const uint16_t* q, const uint16_t* k, const uint16_t* v, const float* g,
                                     const float* beta, const float* state_in, uint16_t* out, float* state_out,
                                     int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                                     int64_t block_size, float scale, void* stream) {
  TRIDA_CHECK(q && k && v && g && beta && state_in && out, TRIDA_ERR_NULL,
              "gdr_block_bidir: q, k, v, g, beta, state_in and out are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hk > 0 && Hv > 0 && Hv % Hk == 0, TRIDA_ERR_ARG, "gdr_block_bidir: bad sizes");
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128 || Dk == 256, TRIDA_ERR_ARG,
              "gdr_block_bidir: Dk must be 32, 64, 128 or 256 (got %lld)", (long long)Dk);
  TRIDA_CHECK(Dv > 0 && Dv % 4 == 0, TRIDA_ERR_ARG, "gdr_block_bidir: Dv must be a multiple of 4");
  TRIDA_CHECK(block_size >= 1 && block_size <= kTC, TRIDA_ERR_ARG, "gdr_block_bidir: block_size in [1, %d]", kTC);
  TRIDA_CHECK(((uintptr_t)q & 15) == 0 && ((uintptr_t)k & 15) == 0 && ((uintptr_t)v & 3) == 0, TRIDA_ERR_ALIGN,
              "gdr_block_bidir: q and k must be 16-byte aligned, v 4-byte aligned");
  TRIDA_CHECK(B * T * Hv < INT32_MAX, TRIDA_ERR_ARG, "gdr_block_bidir: problem too large");
  RecArgs a{q, k, v, g, beta, state_in, out, state_out, nullptr, (int)T, (int)Hk, (int)Hv, (int)Dk,
            (int)Dv, 1, (int)T, scale, (int)block_size, PrepIn{}};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2>(a, (int)B, st);
    case 64: return launch_kpl<4>(a, (int)B, st);
    case 128: return launch_kpl<8>(a, (int)B, st);
    default: return launch_kpl<16>(a, (int)B, st);
  }
}

extern "C" int trida_gdn_fused_layer(const uint16_t* x, const uint16_t* window, const uint16_t* conv_w,
                                     const uint16_t* a_in, const uint16_t* b_in, const float* A_log,
                                     const float* dt_bias, const float* state_in, uint16_t* out, float* state_out,
                                     float* state_clean, uint16_t* k_out, uint16_t* v_out, float* g_out,
                                     float* beta_out, uint16_t* pre_out, uint16_t* window_out, int64_t B,
                                     int64_t T, int64_t Kc, int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                                     int64_t x_sb, int64_t x_st, int64_t ab_sb, int64_t ab_st, int causal_mode,
                                     int64_t num_clean, float scale, const uint16_t* conv_bias,
                                     const int32_t* win_idx, const int32_t* state_idx, float* inter,
                                     const int32_t* inter_idx, int64_t cache_steps, const int32_t* pre_idx,
                                     void* stream) {
  TRIDA_CHECK(x && window && conv_w && a_in && b_in && A_log && dt_bias && state_in && out, TRIDA_ERR_NULL,
              "gdn_fused_layer: x, window, conv_w, a, b, A_log, dt_bias, state_in and out are required");
  TRIDA_CHECK(B > 0 && T > 0 && T <= kTC && Hk > 0 && Hv > 0 && Hv % Hk == 0 && Kc >= 2 && Kc <= kMaxKc,
              TRIDA_ERR_ARG, "gdn_fused_layer: bad sizes B=%lld T=%lld (<= %d) Hk=%lld Hv=%lld Kc=%lld",
              (long long)B, (long long)T, kTC, (long long)Hk, (long long)Hv, (long long)Kc);
  TRIDA_CHECK(Dk == 32 || Dk == 64 || Dk == 128, TRIDA_ERR_ARG, "gdn_fused_layer: Dk must be 32, 64 or 128");
  TRIDA_CHECK(Dv > 0 && Dv % 8 == 0, TRIDA_ERR_ARG, "gdn_fused_layer: Dv must be a multiple of 8");
  TRIDA_CHECK(causal_mode == 1 || causal_mode == 2, TRIDA_ERR_ARG, "gdn_fused_layer: causal_mode is 1 or 2");
  TRIDA_CHECK(num_clean >= 0, TRIDA_ERR_ARG, "gdn_fused_layer: num_clean >= 0");
  TRIDA_CHECK((g_out == nullptr) == (beta_out == nullptr), TRIDA_ERR_ARG,
              "gdn_fused_layer: g_out and beta_out are given together");
  TRIDA_CHECK(state_clean == nullptr || (state_clean != state_in && state_clean != state_out), TRIDA_ERR_ARG,
              "gdn_fused_layer: state_clean must not alias state_in or state_out");
  TRIDA_CHECK(window_out == nullptr || window_out != window, TRIDA_ERR_ARG,
              "gdn_fused_layer: window_out must not alias window");
  const int64_t C = 2 * Hk * Dk + Hv * Dv;
  TRIDA_CHECK(x_st >= C && x_st % 8 == 0 && x_sb % 8 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)window & 15) == 0 &&
                  ((uintptr_t)conv_w & 15) == 0 && ((uintptr_t)k_out & 15) == 0 && ((uintptr_t)pre_out & 15) == 0 &&
                  ((uintptr_t)window_out & 15) == 0,
              TRIDA_ERR_ALIGN, "gdn_fused_layer: x, window, conv_w, k_out, pre_out, window_out 16-byte aligned, x strides in multiples of 8");
  TRIDA_CHECK(B * T * Hv < INT32_MAX && B * T * C < INT32_MAX * 8LL, TRIDA_ERR_ARG, "gdn_fused_layer: problem too large");
  TRIDA_CHECK(inter == nullptr || (cache_steps >= 1 && cache_steps <= INT32_MAX), TRIDA_ERR_ARG,
              "gdn_fused_layer: cache_steps >= 1 with inter");
  TRIDA_CHECK(inter == nullptr || ((uintptr_t)inter & 15) == 0, TRIDA_ERR_ALIGN, "gdn_fused_layer: inter 16-byte aligned");
  TRIDA_CHECK(conv_bias == nullptr || ((uintptr_t)conv_bias & 15) == 0, TRIDA_ERR_ALIGN,
              "gdn_fused_layer: conv_bias 16-byte aligned");
  RecArgs a{nullptr, nullptr, nullptr, nullptr, nullptr, state_in, out, state_out, state_clean, (int)T, (int)Hk,
            (int)Hv, (int)Dk, (int)Dv, causal_mode, (int)num_clean, scale, 0,
            PrepIn{x, window, conv_w, a_in, b_in, A_log, dt_bias, k_out, v_out, g_out, beta_out, pre_out, window_out,
                   conv_bias, win_idx, pre_idx, x_sb, x_st, ab_sb, ab_st, (int)Kc},
            nullptr, state_idx, inter, inter_idx, inter ? (int)cache_steps : 0};
  hipStream_t st = static_cast<hipStream_t>(stream);
  switch (Dk) {
    case 32: return launch_kpl<2, true>(a, (int)B, st);
    case 64: return launch_kpl<4, true>(a, (int)B, st);
    default: return launch_kpl<8, true>(a, (int)B, st);
  }
}
