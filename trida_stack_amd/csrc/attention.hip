// Canvas attention over a bf16 KV cache (draft / verify / mixed masks), MFMA on gfx950.
//
// Query rows of one KV head are the pairs (canvas row t, GQA head g), row m = t * G + g, so the G query
// heads sharing a KV head form one [T*G, D] matrix. Keys p in [0, prefix + T) of the cache; row t sees
// key p when p < prefix (the committed prefix) or, inside the block (j = p - prefix):
//   mask 0 (verify, causal)       j <= t
//   mask 1 (draft, bidirectional) always
//   mask 2 (canvas, mixed)        j <= t for t < n_clean, always for t >= n_clean
//
// attn_partial: workgroup = (sequence, KV head, query tile of <= 128 rows, key split), 8 waves of 16
//   rows each. Per 64-key step, K (XOR-swizzled) and V (row-major, padded rows) are staged in LDS while
//   the next step is loaded into registers; every wave computes S^T = K Q^T for its rows with
//   v_mfma_f32_16x16x32_bf16 (Q and K fragments from LDS), runs the online softmax within the wave, and
//   accumulates O^T += V^T P^T with the V^T fragments read by ds_read_b64_tr_b16.
//   Writes the unnormalised O (bf16), row max and row sum (fp32) of its split. A last tile of <= 16
//   rows can join the tile before it as its extra rows (a canvas of 33 rows x 4 heads = 128 + 4), so
//   the keys stream once for all rows: wave w takes key tile w % 4 of every step for them (an online
//   softmax of its own over those keys) and half w / 4 of their output columns, from the K / V
//   fragments it reads for its own rows; the workgroup merges the four key-tile states at the end.
// attn_combine: merges the splits per row (log-sum-exp weights), applies the optional output gate
//   sigmoid(gate) and writes bf16; attn_combine2 does the same for exactly two splits in one memory round
//   trip per row.
#include <math.h>

#include "common.h"

namespace trida {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kNW = 8;              // waves per workgroup
constexpr int kWR = 16;             // query rows per wave (one MFMA row tile)
constexpr int kMT = kNW * kWR;      // query rows per workgroup, before extra rows
constexpr int kMTX = kMT + kWR;     // with a last tile's <= 16 extra rows
constexpr int kKB = 64;             // keys per step
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxLptSeqs = 256;  // batches up to this size are scheduled longest-first

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  // update_dpp with a defined old value and bound_ctrl: folds into the consuming add / max
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// 2^x with the hardware instruction: exact for the softmax's arguments x <= 0 down to -126, 0 below
// (where the library exp2f would return a denormal)
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

struct AttnArgs {
  const uint16_t* q;        // [B, T, Hq, D]
  const uint16_t* k_cache;  // [B, Hkv, Lmax, D]
  const uint16_t* v_cache;
  const int32_t* prefix;    // [B]
  uint16_t* opart;          // [B, Hkv, QT, S, kMTX, D] bf16
  float* mpart;             // [B, Hkv, QT, S, kMTX]
  float* lpart;
  int T, Hq, Hkv, G, Lmax, S, QT, mask_mode, n_clean;
  float scale_log2;         // softmax scale * log2(e)
  // with one key split (S == 1) the partial kernel writes the final, gated output as the combine would
  const uint16_t* gate;     // row t, head h, dim d at gate + t * gate_st + h * gate_hs + d; or null
  int64_t gate_st, gate_hs;
  uint16_t* out;            // [B, T, Hq, D], or the weight-streaming GEMM's fragment order (frag)
  int frag;
};

// LDS tiles of one 64-key step, 16-byte groups XOR-swizzled so that both the staging writes and the
// MFMA fragment reads touch distinct bank groups:
//   K [key][D]   group g of key k stored at g ^ (k & 7) (16-byte fragment reads, 8 keys per 8 lanes)
//   V [key][D + 16] row-major, rows padded by 32 bytes: the V^T fragments of the P V^T product come from
//                ds_read_b64_tr_b16 (8 bytes of one key per lane, handed out transposed), and the 32 lanes
//                of a half-wave, 8 keys x 32 bytes, then fall on distinct banks; a fragment's address is
//                linear in its column tile (immediate offsets)
template <int D>
__device__ __forceinline__ int k_off(int key, int grp) { return key * D + ((grp ^ (key & 7)) << 3); }
constexpr int kVPad = 16;
template <int D>
__device__ __forceinline__ int v_off(int key, int grp) { return key * (D + kVPad) + (grp << 3); }
// ds_read_b64_tr_b16 (gfx950): in each group of 16 lanes, lane 4 a + b receives element b of the 8-byte
// reads of lanes a, a + 4, a + 8 and a + 12 (in that order). A lane of group g reading key key0 + 4 g +
// (lane % 16) / 4 at columns d0 + 4 (lane % 4) .. + 3 thus receives V[key0 + 4 g + j][d0 + lane % 16] for
// j = 0..3: four keys of its V^T row, in the k slots of the MFMA's A operand.
template <int D>
__device__ __forceinline__ s16x4 vt_frag4(const uint16_t* sV, int key0, int d0, int l) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int key = key0 + 4 * (l / 16) + (l % 16) / 4, col = d0 + 4 * (l % 4);
  const uint16_t* p = sV + v_off<D>(key, col / 8) + col % 8;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uint32_t)(uintptr_t)p);
}

// Workgroup = (sequence, KV head, query tile of kMT rows, key split); 8 waves, wave w owns rows
// [16 w, 16 w + 16) of the tile. Per 64-key step: K and V^T are staged in LDS (the next step's K / V
// are loaded into registers meanwhile) and the wave forms the transposed products S^T = K Q^T and
// O^T += V^T P^T on v_mfma_f32_16x16x32_bf16, so lane l holds 16 scores and 256 / 4 output values of
// one query row (l % 16): the online softmax of a row is the lane's own, completed across its four
// lane groups by two xor exchanges, and its probabilities are, as computed, the B operand of the
// product with V (a 32-key block takes slots 8 g + j = keys 32 kk + 4 g + j and 32 kk + 16 + 4 g + j - 4,
// which is where the two key tiles' accumulators put them). O is rescaled only when a row's running max
// moved. Writes the unnormalised O, the row max (log2 domain) and the row sum of its split.
// Extra rows (the last tile's kMT .. kMT + 15): wave w forms the 16 keys x 16 rows of key tile w % 4 of
// their S^T with the K fragments of its own product (the extra rows' Q from LDS), runs an online softmax
// over the keys it sees this way, and accumulates columns [D/2 (w / 4), D/2 (w / 4 + 1)) of their O^T on
// v_mfma_f32_16x16x16_bf16, whose B operand is the S^T accumulator layout as it stands (A: 4 keys of a
// V^T row from the staged tile). No barrier inside a step; after the last one the waves of each column
// half merge their four key tiles' states through LDS in key-tile order.
template <int D>
__global__ __launch_bounds__(kNW* kWave) void attn_partial_kernel(AttnArgs a) {
  constexpr int KC = D / 32;         // 32-wide k-chunks of the head dim (QK^T)
  constexpr int CT = D / 16;         // 16-column tiles of O
  constexpr int GPR = D / 8;         // 16-byte groups per K row
  constexpr int NT = kNW * kWave;
  constexpr int NKG = kKB * GPR / NT;  // K groups staged per thread
  constexpr int XH = CT / 2;  // O^T column tiles of the extra rows per wave (half of them)
  __shared__ __align__(16) uint16_t sQ[kMT * D];  // [row][D], groups swizzled by row & 7 (as K)
  __shared__ __align__(16) uint16_t sQx[kWR * D];  // the extra rows, the same layout
  __shared__ __align__(16) uint16_t sK[kKB * D];
  __shared__ __align__(16) uint16_t sV[kKB * (D + kVPad)];
  __shared__ float sXm[kNW][kWR], sXl[kNW][kWR];  // the extra rows' per-wave running max and sum

  const int tid = threadIdx.x, w = tid / kWave, l = tid % kWave;
  const int per_pair = a.S * a.QT;                  // workgroups per (sequence, KV head)
  const int npair = (int)gridDim.x / per_pair, nseq = npair / a.Hkv;
  int b, hk, s, qt;
  if (nseq > 1 && nseq <= kMaxLptSeqs && npair % kXcds == 0) {
    // ragged batches: longest sequences first. Workgroups reach the XCDs round-robin in block order,
    // so (sequence, KV head) pairs are dealt to the XCDs in descending prefix length, each pair's
    // workgroups consecutive on one XCD (its query tiles share the keys in that L2); the longest pairs
    // start in the first wave of workgroups instead of wherever their batch index put them.
    __shared__ int s_len[kMaxLptSeqs];
    __shared__ int s_seq;
    const int x = (int)blockIdx.x % kXcds, j = (int)blockIdx.x / kXcds;
    const int pr = (j / per_pair) * kXcds + x;  // pair rank
    const int wi = j % per_pair;
    qt = wi % a.QT;
    s = wi / a.QT;
    hk = pr % a.Hkv;
    const int r = pr / a.Hkv;  // sequence rank: prefix length descending, batch index ascending
    for (int c = tid; c < nseq; c += kNW * kWave) s_len[c] = a.prefix[c];
    __syncthreads();
    for (int c = tid; c < nseq; c += kNW * kWave) {
      const int lc = s_len[c];
      int rank = 0;
      for (int o = 0; o < nseq; ++o) rank += (s_len[o] > lc) | ((s_len[o] == lc) & (o < c));
      if (rank == r) s_seq = c;
    }
    __syncthreads();
    b = s_seq;
  } else {
    // query tiles of one (split, kv head) read the same keys: innermost, and on one XCD
    int idx = xcd_major(blockIdx.x, gridDim.x);
    qt = idx % a.QT;
    idx /= a.QT;
    s = idx % a.S;
    idx /= a.S;
    hk = idx % a.Hkv;
    b = idx / a.Hkv;
  }
  const int M = a.T * a.G;
  const int m0 = qt * kMT;
  // the tile's rows: kMT, or for the last tile all that remain (<= kMTX: nx extra rows past kMT)
  const int rows = qt == a.QT - 1 ? M - m0 : kMT;
  const int nx = max(rows - kMT, 0);  // block-uniform
  // a prefix past the cache capacity (a caller's overlong decode) is clamped so that every key read
  // stays inside this sequence's [Lmax, D] rows
  const int prefix = min(max(a.prefix[b], 0), a.Lmax - a.T);
  const int nk = prefix + a.T;
  const int nblk = (nk + kKB - 1) / kKB;
  const int bps = (nblk + a.S - 1) / a.S;
  const int kb0 = s * bps;
  // the last query row of the tile bounds the keys any row can see under the causal masks
  const int t_last = (m0 + rows - 1) / a.G;
  const int kmax = (a.mask_mode == 1 || (a.mask_mode == 2 && t_last >= a.n_clean)) ? nk : min(nk, prefix + t_last + 1);
  const int kb1 = min(min(nblk, kb0 + bps), (kmax + kKB - 1) / kKB);

  const int64_t pbase = ((((int64_t)b * a.Hkv + hk) * a.QT + qt) * a.S + s);
  if (kb0 >= kb1) {
    // no key of this split is visible to the tile: only the (empty) row stats are written and the
    // combine skips the split without reading its O (never with one split: its keys start at 0 and every
    // row sees at least its own)
    for (int r = tid; r < rows; r += NT) {
      a.mpart[pbase * kMTX + r] = -INFINITY;
      a.lpart[pbase * kMTX + r] = 0.f;
    }
    return;
  }
  const uint16_t* kh = a.k_cache + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;
  const uint16_t* vh = a.v_cache + ((int64_t)b * a.Hkv + hk) * a.Lmax * D;

  // ---- prefetch registers: K and V groups (coalesced rows)
  u32x4 kreg[NKG], vreg[NKG];
  auto load_step = [&](int kb) {
    const int key0 = kb * kKB;
#pragma unroll
    for (int j = 0; j < NKG; ++j) {
      const int gi = tid + j * NT;
      const int key = min(key0 + gi / GPR, nk - 1);
      kreg[j] = *reinterpret_cast<const u32x4*>(kh + (int64_t)key * D + (gi % GPR) * 8);
      vreg[j] = *reinterpret_cast<const u32x4*>(vh + (int64_t)key * D + (gi % GPR) * 8);
    }
  };
  // the first step's K / V loads go out with the Q loads: one memory latency for both
  load_step(kb0);

  // ---- the tile's Q rows into LDS (padding rows zero); read back as A fragments every step. Every
  // load of the tile is issued before the first store, so the staging costs one memory latency.
  {
    constexpr int QPT = kMT * GPR / NT;  // 16-byte pieces per thread
    static_assert(kWR * GPR <= NT, "one piece of the extra rows per thread");
    u32x4 qv[QPT], qx = u32x4{0u, 0u, 0u, 0u};
    auto q_at = [&](int m, int grp) {
      const int t = m / a.G, g = m % a.G;
      return *reinterpret_cast<const u32x4*>(a.q + (((int64_t)b * a.T + t) * a.Hq + hk * a.G + g) * D + grp * 8);
    };
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
      const int gi = tid + j * NT;
      qv[j] = q_at(m0 + min(gi / GPR, rows - 1), gi % GPR);
    }
    if (nx > 0 && tid < kWR * GPR) qx = q_at(m0 + kMT + min(tid / GPR, nx - 1), tid % GPR);
#pragma unroll
    for (int j = 0; j < QPT; ++j) {
      const int gi = tid + j * NT;
      const int r = gi / GPR, grp = gi % GPR;
      *reinterpret_cast<u32x4*>(&sQ[k_off<D>(r, grp)]) = r < rows ? qv[j] : u32x4{0u, 0u, 0u, 0u};
    }
    if (nx > 0 && tid < kWR * GPR)
      *reinterpret_cast<u32x4*>(&sQx[k_off<D>(tid / GPR, tid % GPR)]) = tid / GPR < nx ? qx : u32x4{0u, 0u, 0u, 0u};
  }

  auto stage_step = [&]() {
#pragma unroll
    for (int j = 0; j < NKG; ++j) {
      const int gi = tid + j * NT;
      *reinterpret_cast<u32x4*>(&sK[k_off<D>(gi / GPR, gi % GPR)]) = kreg[j];
      *reinterpret_cast<u32x4*>(&sV[v_off<D>(gi / GPR, gi % GPR)]) = vreg[j];
    }
  };

  // o[ct] holds O[row][16 ct + 4 (l / 16) + e] of this lane's query row 16 w + l % 16
  f32x4 o[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) o[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  // the keys the lane's row sees are exactly [0, klim): the whole prefix, then the block keys its mask
  // allows (a prefix of the block for the causal rows, all of it for the others)
  int klim;
  {
    const int t = (m0 + w * kWR + (l % 16)) / a.G;
    const bool all = a.mask_mode == 1 || (a.mask_mode == 2 && t >= a.n_clean);
    klim = all ? nk : min(nk, prefix + t + 1);
  }
  const int g4 = 4 * (l / 16);

  // ---- mask, scale and online softmax of one step's scores sc (keys 16 kt + g4 + e of the lane's row, which
  // sees the keys below lim) against the row's running max m and sum lsum; returns the probabilities as the
  // B fragments of the two 32-key blocks in pb and the rescale factor of the row's O. The mask applies only
  // on steps that reach the block keys or the cache end (uniform)
  auto softmax_step = [&](f32x4 (&sc)[4], int key0, int lim, float& m, float& lsum, u32x4 (&pb)[2]) {
    const bool edge = key0 + kKB > prefix || key0 + kKB > nk;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[kt][e] *= a.scale_log2;
    if (edge) {
#pragma unroll
      for (int kt = 0; kt < 4; ++kt)
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[kt][e] = key0 + 16 * kt + g4 + e < lim ? sc[kt][e] : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3]));
#pragma unroll
    for (int kt = 1; kt < 4; ++kt) mx = fmaxf(mx, fmaxf(fmaxf(sc[kt][0], sc[kt][1]), fmaxf(sc[kt][2], sc[kt][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_hw(m - m_use);
    m = m_new;
    float ps = 0.f;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      float p[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        p[e] = exp2_hw(sc[2 * kk][e] - m_use);
        p[4 + e] = exp2_hw(sc[2 * kk + 1][e] - m_use);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ps += p[e];
      pb[kk] = u32x4{f2bf2(p[0], p[1]), f2bf2(p[2], p[3]), f2bf2(p[4], p[5]), f2bf2(p[6], p[7])};
    }
    ps += __shfl_xor(ps, 16, kWave);
    ps += __shfl_xor(ps, 32, kWave);
    lsum = lsum * alpha + ps;
    return alpha;
  };

  // the extra rows: this wave's key tile and column half, its running max / sum over the keys of that tile,
  // its O^T column tiles, and the keys the lanes' rows see
  const int ktx = w % 4, dh = w / 4;
  f32x4 ox[XH];
#pragma unroll
  for (int j = 0; j < XH; ++j) ox[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mx_run = -INFINITY, lx_run = 0.f;
  int klim_x = 0;
  if (nx > 0) {
    const int t = (m0 + kMT + min(l % 16, nx - 1)) / a.G;
    const bool all = a.mask_mode == 1 || (a.mask_mode == 2 && t >= a.n_clean);
    klim_x = all ? nk : min(nk, prefix + t + 1);
  }
  // one step of the extra rows: sx = S^T of key tile ktx (keys 16 ktx + g4 + e of the lane's row)
  auto extra_step = [&](f32x4 sx, int key0) {
    const bool edge = key0 + kKB > prefix || key0 + kKB > nk;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sx[e] *= a.scale_log2;
      if (edge) sx[e] = key0 + 16 * ktx + g4 + e < klim_x ? sx[e] : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sx[0], sx[1]), fmaxf(sx[2], sx[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(mx_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_hw(mx_run - m_use);
    mx_run = m_new;
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = exp2_hw(sx[e] - m_use);
    float ps = (p[0] + p[1]) + (p[2] + p[3]);
    ps += __shfl_xor(ps, 16, kWave);
    ps += __shfl_xor(ps, 32, kWave);
    lx_run = lx_run * alpha + ps;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int j = 0; j < XH; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) ox[j][e] *= alpha;
    }
    const s16x4 pf = __builtin_bit_cast(s16x4, u32x2{f2bf2(p[0], p[1]), f2bf2(p[2], p[3])});
    // V^T row (dh XH + j) 16 + l % 16, keys 16 ktx + g4 .. + 3
#pragma unroll
    for (int j = 0; j < XH; ++j) {
      const s16x4 vf = vt_frag4<D>(sV, 16 * ktx, (dh * XH + j) * 16, l);
      ox[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf, pf, ox[j], 0, 0, 0);
    }
  };

  for (int kb = kb0; kb < kb1; ++kb) {
    const int key0 = kb * kKB;
    __syncthreads();  // the previous step's tiles are consumed
    stage_step();
    __syncthreads();
    if (kb + 1 < kb1) load_step(kb + 1);  // in flight during this step's MFMAs
    // a wave with no row of the tile (a last tile of fewer rows) only helps stage the keys: its fragment
    // reads and MFMAs would be on padding (wave-uniform; no barrier inside)
    if (w * kWR >= rows) continue;
    // ---- S^T = K Q^T: keys 16 kt + 4 (l / 16) + e of this lane's query row (4 key tiles), and key tile ktx
    // of the extra rows
    f32x4 sacc[4], sx = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) sacc[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const bf16x8 qf = as_bf16x8(*reinterpret_cast<const u32x4*>(&sQ[k_off<D>(w * kWR + (l % 16), kc * 4 + l / 16)]));
      bf16x8 kfx = qf;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const bf16x8 kf =
            as_bf16x8(*reinterpret_cast<const u32x4*>(&sK[k_off<D>(kt * 16 + (l % 16), kc * 4 + l / 16)]));
        sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf, sacc[kt], 0, 0, 0);
        if (kt == ktx) kfx = kf;
      }
      if (nx > 0) {  // block-uniform
        const bf16x8 qxf = as_bf16x8(*reinterpret_cast<const u32x4*>(&sQx[k_off<D>(l % 16, kc * 4 + l / 16)]));
        sx = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kfx, qxf, sx, 0, 0, 0);
      }
    }
    u32x4 pb[2];
    const float alpha = softmax_step(sacc, key0, klim, m_run, l_run, pb);
    // rescale O only when some row's running max moved (rare once the max settles)
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int e = 0; e < 4; ++e) o[ct][e] *= alpha;
    }
    // ---- O^T += V^T P^T (V^T fragments by transposed LDS reads, in the slot order of the probabilities:
    // keys 32 kk + g4 .. + 3, then 32 kk + 16 + g4 .. + 3)
#pragma unroll
    for (int kk = 0; kk < kKB / 32; ++kk) {
      const bf16x8 pf = as_bf16x8(pb[kk]);
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const s16x4 v0 = vt_frag4<D>(sV, 32 * kk, ct * 16, l), v1 = vt_frag4<D>(sV, 32 * kk + 16, ct * 16, l);
        const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
        const bf16x8 vf = as_bf16x8(u32x4{w0.x, w0.y, w1.x, w1.y});
        o[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[ct], 0, 0, 0);
      }
    }
    if (nx > 0) extra_step(sx, key0);
  }
  if (nx > 0) {
    // merge the extra rows' four key-tile states of each column half into its first wave (w % 4 == 0), in
    // key-tile order; the K / V tiles and Q are no longer read, and sQ holds the other waves' O^T tiles
    __syncthreads();
    f32x4* xo = reinterpret_cast<f32x4*>(sQ);  // [column half][key tile 1..3][XH][lane]
    static_assert(2 * 3 * XH * kWave * 16 <= kMT * D * 2, "the merge's O^T tiles fit in sQ");
    if (ktx > 0) {
#pragma unroll
      for (int j = 0; j < XH; ++j) xo[((dh * 3 + ktx - 1) * XH + j) * kWave + l] = ox[j];
    }
    if (l < kWR) {
      sXm[w][l] = mx_run;
      sXl[w][l] = lx_run;
    }
    __syncthreads();
    if (ktx == 0) {
      const int rr = l % 16;
      float mm = mx_run;
#pragma unroll
      for (int k = 1; k < 4; ++k) mm = fmaxf(mm, sXm[dh * 4 + k][rr]);
      const float m_use = mm == -INFINITY ? 0.f : mm;
      const float e0 = exp2_hw(mx_run - m_use);
      float ls = lx_run * e0;
#pragma unroll
      for (int j = 0; j < XH; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) ox[j][e] *= e0;
#pragma unroll
      for (int k = 1; k < 4; ++k) {
        const float ek = exp2_hw(sXm[dh * 4 + k][rr] - m_use);
        ls += ek * sXl[dh * 4 + k][rr];
#pragma unroll
        for (int j = 0; j < XH; ++j) {
          const f32x4 v = xo[((dh * 3 + k - 1) * XH + j) * kWave + l];
#pragma unroll
          for (int e = 0; e < 4; ++e) ox[j][e] += ek * v[e];
        }
      }
      mx_run = mm;
      lx_run = ls;
    }
  }
  const int r = w * kWR + (l % 16), rx = kMT + (l % 16);  // the lane's row and extra row of the tile
  const bool own = r < rows, extra = ktx == 0 && l % 16 < nx;
  if (a.S == 1) {
    // ---- the only split: O / l, rounded to bf16, then the gate, exactly as the combine computes it
    auto emit = [&](int rr, float lsum, const f32x4& v, int ct) {
      const int m = m0 + rr, t = m / a.G, hq = hk * a.G + m % a.G;
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      const int c = ct * 16 + g4;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = bf2f(f2bf(v[e])) * inv;
      if (a.gate) {
        const u32x2 gw = *reinterpret_cast<const u32x2*>(a.gate + ((int64_t)b * a.T + t) * a.gate_st +
                                                         (int64_t)hq * a.gate_hs + c);
        const float gv[4] = {__uint_as_float(gw.x << 16), __uint_as_float(gw.x & 0xffff0000u),
                             __uint_as_float(gw.y << 16), __uint_as_float(gw.y & 0xffff0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = bf2f(f2bf(y[e])) * (1.f / (1.f + __expf(-gv[e])));
      }
      uint16_t* dst = a.frag ? a.out + ws_frag_off(b * a.T + t, (int64_t)hq * D + c)
                             : a.out + (((int64_t)b * a.T + t) * a.Hq + hq) * D + c;
      *reinterpret_cast<u32x2*>(dst) = u32x2{f2bf2(y[0], y[1]), f2bf2(y[2], y[3])};
    };
    if (own) {
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) emit(r, l_run, o[ct], ct);
    }
    if (extra) {
#pragma unroll
      for (int j = 0; j < XH; ++j) emit(rx, lx_run, ox[j], dh * XH + j);
    }
    return;
  }
  // ---- write this split's unnormalised O (bf16: half the partial traffic; 8-byte row pieces) and row
  // stats (fp32)
  uint16_t* op = a.opart + pbase * kMTX * D;
  auto park = [&](int rr, const f32x4& v, int ct) {
    *reinterpret_cast<u32x2*>(&op[(int64_t)rr * D + ct * 16 + g4]) = u32x2{f2bf2(v[0], v[1]), f2bf2(v[2], v[3])};
  };
  if (own) {
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) park(r, o[ct], ct);
    if (l < 16) {
      a.mpart[pbase * kMTX + r] = m_run;
      a.lpart[pbase * kMTX + r] = l_run;
    }
  }
  if (extra) {
#pragma unroll
    for (int j = 0; j < XH; ++j) park(rx, ox[j], dh * XH + j);
    if (w == 0 && l < 16) {
      a.mpart[pbase * kMTX + rx] = mx_run;
      a.lpart[pbase * kMTX + rx] = lx_run;
    }
  }
}

struct CombineArgs {
  const uint16_t* opart;  // bf16
  const float* mpart;
  const float* lpart;
  const uint16_t* gate;  // row t, head h, dim d at gate + t * gate_st + h * gate_hs + d; or null
  uint16_t* out;         // [B, T, Hq, D], or the rows [B * T, Hq * D] in the weight-streaming GEMM's
                         // fragment order (frag)
  int T, Hq, Hkv, G, D, S, QT;
  int64_t gate_st, gate_hs;
  int frag;
};

// Block = a group of RB = 512 / D rows of one (sequence, KV head); thread = (row, 4 output columns).
// The split weights exp2(m_s - max) / sum of the group's rows are computed once into LDS; each thread
// then sums the O rows of the non-empty splits in split order. Every phase issues its loads together
// (clamped, unconditional): the listing's row statistics, a row's max and sum (one pass over m and l),
// 16 splits' O rows at a time, and the gate first of all, so the combine costs a few memory round trips
// instead of one per four splits.
constexpr int kMaxSplits = 256;
constexpr int kOB = 16;  // O rows in flight per thread

constexpr int kCT = 128;  // combine threads per block (2 waves): 2 rows of d 256 per block, so a
                          // batch-1 canvas (132 rows per KV head) spreads over the CUs
template <int D>
__global__ __launch_bounds__(kCT) void attn_combine_kernel(CombineArgs a) {
  constexpr int PER_ROW = D / 4;
  constexpr int RB = kCT / PER_ROW;  // rows per block: 2 (D=256), 4 (D=128), 8 (D=64)
  constexpr int NWV = kCT / kWave;
  constexpr int LP = kMaxSplits / kCT;  // splits per thread in the listing
  __shared__ float s_w[RB][kMaxSplits];  // rows of the group x listed splits
  __shared__ float s_inv[RB];
  __shared__ int s_list[kMaxSplits];
  __shared__ int s_cnt[LP][NWV];
  const int M = a.T * a.G;
  const int b = blockIdx.y / a.Hkv, hk = blockIdx.y % a.Hkv;
  const int m0 = blockIdx.x * RB;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int64_t pair = (int64_t)b * a.Hkv + hk;
  // this thread's output element group (rows past M compute on row M - 1 and store nothing)
  const int i = tid / PER_ROW;
  const int m = m0 + i;
  const int mc = min(m, M - 1);
  const int c = (tid % PER_ROW) * 4;
  const int t = mc / a.G, g = mc % a.G, hq = hk * a.G + g;
  u32x2 gw = {0u, 0u};
  if (a.gate)
    gw = *reinterpret_cast<const u32x2*>(a.gate + ((int64_t)b * a.T + t) * a.gate_st + (int64_t)hq * a.gate_hs + c);
  // list, in split order, the splits with a visible key for some row of the group (splits tid and
  // tid + kCT of each thread, S <= 256; wave ballots give each listed split its position)
  bool any[LP];
  {
    float mv[LP][RB];
#pragma unroll
    for (int q = 0; q < LP; ++q) {
      const int sp = min(tid + q * kCT, a.S - 1);
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int mr = min(m0 + r, M - 1);
        const int tq = min(mr / kMT, a.QT - 1);
        mv[q][r] = a.mpart[((pair * a.QT + tq) * a.S + sp) * kMTX + (mr - tq * kMT)];
      }
    }
#pragma unroll
    for (int q = 0; q < LP; ++q) {
      any[q] = false;
#pragma unroll
      for (int r = 0; r < RB; ++r) any[q] |= m0 + r < M && mv[q][r] != -INFINITY;
      any[q] &= tid + q * kCT < a.S;
    }
  }
  unsigned long long mask[LP];
#pragma unroll
  for (int q = 0; q < LP; ++q) {
    mask[q] = __ballot(any[q]);
    if (lane == 0) s_cnt[q][wave] = __popcll(mask[q]);
  }
  __syncthreads();
  int ns = 0;
#pragma unroll
  for (int q = 0; q < LP; ++q) {
    int off = ns;
    for (int w = 0; w < wave; ++w) off += s_cnt[q][w];
    if (any[q]) s_list[off + __popcll(mask[q] & ((1ull << lane) - 1ull))] = tid + q * kCT;
    for (int w = 0; w < NWV; ++w) ns += s_cnt[q][w];
  }
  __syncthreads();
  // per row: max, weights and 1 / sum (one wave per row, lanes over the listed splits; m and l of a
  // lane's splits loaded together)
  for (int ri = wave; ri < RB; ri += NWV) {
    const int mr = min(m0 + ri, M - 1);
    const int tq = min(mr / kMT, a.QT - 1);  // the last tile holds its extra rows past kMT
    const int64_t bs = (pair * a.QT + tq) * a.S;
    const int r = mr - tq * kMT;
    constexpr int JU = kMaxSplits / kWave;  // listed splits per lane, at most
    float mj[JU], lj[JU];
#pragma unroll
    for (int u = 0; u < JU; ++u) {
      const int j = lane + u * kWave;
      if (u * kWave < ns) {  // uniform
        const int sj = s_list[min(j, ns - 1)];
        mj[u] = a.mpart[(bs + sj) * kMTX + r];
        lj[u] = a.lpart[(bs + sj) * kMTX + r];
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < JU; ++u)
      if (u * kWave < ns && lane + u * kWave < ns) mx = fmaxf(mx, mj[u]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, kWave));
    const float m_use = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < JU; ++u) {
      const int j = lane + u * kWave;
      if (u * kWave < ns && j < ns) {
        const float w = exp2f(mj[u] - m_use);
        s_w[ri][j] = w;
        lsum += w * lj[u];
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o, kWave);
    if (lane == 0) s_inv[ri] = lsum > 0.f ? 1.f / lsum : 0.f;
  }
  __syncthreads();
  const int tqc = min(mc / kMT, a.QT - 1);
  const int64_t bs = (pair * a.QT + tqc) * a.S;
  const uint16_t* obase = a.opart + (int64_t)(mc - tqc * kMT) * D + c;
  const int64_t sstride = (int64_t)kMTX * D;  // elements between consecutive splits
  auto ld4 = [](const uint16_t* p) {  // 4 bf16 -> fp32
    const u32x2 w = *reinterpret_cast<const u32x2*>(p);
    return f32x4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xffff0000u), __uint_as_float(w.y << 16),
                 __uint_as_float(w.y & 0xffff0000u)};
  };
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < ns; j0 += kOB) {
    f32x4 x[kOB];
#pragma unroll
    for (int u = 0; u < kOB; ++u) x[u] = ld4(obase + (bs + s_list[min(j0 + u, ns - 1)]) * sstride);
#pragma unroll
    for (int u = 0; u < kOB; ++u)
      if (j0 + u < ns) acc += s_w[i < RB ? i : 0][j0 + u] * x[u];  // uniform bound; split order kept
  }
  if (i >= RB || m >= M) return;
  const float inv = s_inv[i];
  float y[4] = {acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv};
  if (a.gate) {
    const float gv[4] = {__uint_as_float(gw.x << 16), __uint_as_float(gw.x & 0xffff0000u), __uint_as_float(gw.y << 16),
                         __uint_as_float(gw.y & 0xffff0000u)};
#pragma unroll
    for (int u = 0; u < 4; ++u)  // the attention output is rounded to bf16 before the gate, as torch does
      y[u] = bf2f(f2bf(y[u])) * (1.f / (1.f + __expf(-gv[u])));
  }
  uint16_t* dst = a.frag ? a.out + ws_frag_off(b * a.T + t, (int64_t)hq * D + c)
                         : a.out + (((int64_t)b * a.T + t) * a.Hq + hq) * D + c;
  *reinterpret_cast<u32x2*>(dst) = u32x2{f2bf2(y[0], y[1]), f2bf2(y[2], y[3])};
}

// Two splits (batches of sequences): thread = (row, 4 output columns), 256 threads = 1024 / D rows. Every
// load of a row -- both splits' statistics and O pieces, the gate -- is issued at once, so the combine is
// one memory round trip. The arithmetic is attn_combine_kernel's: a split whose row sees no key (m = -inf)
// adds nothing (and its O, which an empty split never wrote, is not used); with two terms the order of the
// sums cannot differ, so the results are bitwise equal.
constexpr int kC2T = 256;
bool combine_general = false;  // trida_attn_set_combine_general: the general combine for two splits too
template <int D>
__global__ __launch_bounds__(kC2T) void attn_combine2_kernel(CombineArgs a) {
  constexpr int PER_ROW = D / 4;
  constexpr int RB = kC2T / PER_ROW;
  const int M = a.T * a.G;
  const int b = blockIdx.y / a.Hkv, hk = blockIdx.y % a.Hkv;
  const int tid = threadIdx.x, i = tid / PER_ROW, c = (tid % PER_ROW) * 4;
  const int m = blockIdx.x * RB + i;
  if (m >= M) return;  // no barrier in this kernel
  const int t = m / a.G, g = m % a.G, hq = hk * a.G + g;
  const int64_t pair = (int64_t)b * a.Hkv + hk;
  const int tq = min(m / kMT, a.QT - 1);  // the last tile holds its extra rows past kMT
  const int64_t bs = (pair * a.QT + tq) * 2;
  const int r = m - tq * kMT;
  u32x2 gw = {0u, 0u};
  if (a.gate)
    gw = *reinterpret_cast<const u32x2*>(a.gate + ((int64_t)b * a.T + t) * a.gate_st + (int64_t)hq * a.gate_hs + c);
  const float m0 = a.mpart[bs * kMTX + r], m1 = a.mpart[(bs + 1) * kMTX + r];
  const float l0 = a.lpart[bs * kMTX + r], l1 = a.lpart[(bs + 1) * kMTX + r];
  const uint16_t* o0 = a.opart + (bs * kMTX + r) * D + c;
  const u32x2 x0w = *reinterpret_cast<const u32x2*>(o0);
  const u32x2 x1w = *reinterpret_cast<const u32x2*>(o0 + (int64_t)kMTX * D);
  const float mx = fmaxf(m0, m1);
  const float m_use = mx == -INFINITY ? 0.f : mx;
  const bool u0 = m0 != -INFINITY, u1 = m1 != -INFINITY;
  const float w0 = u0 ? exp2f(m0 - m_use) : 0.f, w1 = u1 ? exp2f(m1 - m_use) : 0.f;
  float lsum;
  {
#pragma clang fp contract(off)
    lsum = w0 * l0 + w1 * l1;  // each product rounded, as the lanes of the general combine's sum hold them
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  const float x0[4] = {__uint_as_float(x0w.x << 16), __uint_as_float(x0w.x & 0xffff0000u), __uint_as_float(x0w.y << 16),
                       __uint_as_float(x0w.y & 0xffff0000u)};
  const float x1[4] = {__uint_as_float(x1w.x << 16), __uint_as_float(x1w.x & 0xffff0000u), __uint_as_float(x1w.y << 16),
                       __uint_as_float(x1w.y & 0xffff0000u)};
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float acc = 0.f;
    if (u0) acc = fmaf(w0, x0[e], acc);
    if (u1) acc = fmaf(w1, x1[e], acc);
    y[e] = acc * inv;
  }
  if (a.gate) {
    const float gv[4] = {__uint_as_float(gw.x << 16), __uint_as_float(gw.x & 0xffff0000u), __uint_as_float(gw.y << 16),
                         __uint_as_float(gw.y & 0xffff0000u)};
#pragma unroll
    for (int e = 0; e < 4; ++e)  // the attention output is rounded to bf16 before the gate, as torch does
      y[e] = bf2f(f2bf(y[e])) * (1.f / (1.f + __expf(-gv[e])));
  }
  uint16_t* dst = a.frag ? a.out + ws_frag_off(b * a.T + t, (int64_t)hq * D + c)
                         : a.out + (((int64_t)b * a.T + t) * a.Hq + hq) * D + c;
  *reinterpret_cast<u32x2*>(dst) = u32x2{f2bf2(y[0], y[1]), f2bf2(y[2], y[3])};
}

// Splits per (sequence, KV head, query tile): as many as keep the grid within one workgroup per CU
// (a workgroup holds a CU's LDS), at least one key block each. Measured at batch 1 (33 canvas rows,
// 16 / 4 heads, d 256): 2200 keys 30.0 -> 25 us, 8192 keys 54.2 -> 40 us against splits of >= 4 key
// blocks; a grid just past the CU count (33 splits) runs a ragged second round and is slower.
// When the query tiles alone fill the CUs (a batch of sequences), two splits per tile, so that the
// longest sequences of a ragged batch are not one workgroup's serial walk over their keys (64 sequences
// of 512-4096 keys, 32 rows x 4 heads: 245 -> 201 us).
constexpr int64_t kCUs = 256;
int64_t plan_splits(int64_t B, int64_t Hkv, int64_t QT, int64_t max_keys, int64_t splits) {
  if (splits > 0) return splits;
  const int64_t nblk = cdiv(max_keys, kKB);
  if (B * Hkv * QT >= kCUs) return std::max<int64_t>(1, std::min<int64_t>(2, nblk));
  int64_t s = kCUs / (B * Hkv * QT);
  if (s > nblk) s = nblk;
  if (s > kMaxSplits) s = kMaxSplits;
  return s < 1 ? 1 : s;
}

// Query tiles of M rows per (sequence, KV head): kMT rows each. A last one of <= 16 rows joins the tile
// before it as its extra rows when its own workgroups would not fit beside the others on the CUs (a batch
// of sequences; 64 x 33 rows x 4 heads, 512-4096 keys: 277 -> 243 us). Where they fit (batch 1) they run
// on otherwise idle CUs and the extra rows' work would only lengthen the full tile's (23.1 -> 25.5 us).
int64_t query_tiles(int64_t B, int64_t Hkv, int64_t M) {
  const int64_t qt = cdiv(M, kMT);
  return qt > 1 && M - (qt - 1) * kMT <= kWR && B * Hkv * qt > kCUs ? qt - 1 : qt;
}

}  // namespace
}  // namespace trida

using namespace trida;

extern "C" int64_t trida_attn_canvas_scratch_bytes(int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                                   int64_t max_keys, int64_t splits) {
  if (B <= 0 || T <= 0 || Hkv <= 0 || Hq % Hkv || D <= 0) return 0;
  const int64_t QT = query_tiles(B, Hkv, T * (Hq / Hkv));
  const int64_t S = plan_splits(B, Hkv, QT, max_keys, splits);
  const int64_t slots = B * Hkv * QT * S;
  return align_up(slots * kMTX * D * 2, 256) + 2 * align_up(slots * kMTX * 4, 256);
}

namespace {
int attn_canvas_run(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* prefix_len,
                    const uint16_t* gate, int64_t gate_row_stride, int64_t gate_head_stride, uint16_t* out, bool frag,
                    int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D, int64_t Lmax, int mask_mode,
                    int64_t n_clean, float scale, int64_t max_keys, int64_t splits, void* scratch,
                    int64_t scratch_bytes, void* stream) {
  TRIDA_CHECK(q && k_cache && v_cache && prefix_len && out && scratch, TRIDA_ERR_NULL,
              "attn_canvas: q, k_cache, v_cache, prefix_len, out and scratch are required");
  TRIDA_CHECK(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0 && Lmax >= T, TRIDA_ERR_ARG,
              "attn_canvas: bad sizes B=%lld T=%lld Hq=%lld Hkv=%lld Lmax=%lld", (long long)B, (long long)T,
              (long long)Hq, (long long)Hkv, (long long)Lmax);
  TRIDA_CHECK(D == 64 || D == 128 || D == 256, TRIDA_ERR_ARG, "attn_canvas: head dim must be 64, 128 or 256");
  TRIDA_CHECK(mask_mode >= 0 && mask_mode <= 2, TRIDA_ERR_ARG, "attn_canvas: mask_mode is 0, 1 or 2");
  TRIDA_CHECK(((((uintptr_t)q) | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) == 0,
              TRIDA_ERR_ALIGN, "attn_canvas: q, caches and out must be 16-byte aligned");
  TRIDA_CHECK(gate == nullptr || (gate_head_stride >= D && gate_row_stride >= Hq * gate_head_stride - (gate_head_stride - D)),
              TRIDA_ERR_ARG, "attn_canvas: gate strides");
  const int64_t G = Hq / Hkv;
  const int64_t QT = query_tiles(B, Hkv, T * G);
  const int64_t S = plan_splits(B, Hkv, QT, max_keys > 0 ? max_keys : Lmax, splits);
  TRIDA_CHECK(S >= 1 && S <= kMaxSplits, TRIDA_ERR_ARG, "attn_canvas: 1..%d key splits", kMaxSplits);
  const int64_t need = trida_attn_canvas_scratch_bytes(B, T, Hq, Hkv, D, max_keys > 0 ? max_keys : Lmax, S);
  TRIDA_CHECK(scratch_bytes >= need, TRIDA_ERR_WORKSPACE, "attn_canvas: scratch %lld < %lld bytes",
              (long long)scratch_bytes, (long long)need);
  const int64_t slots = B * Hkv * QT * S;
  TRIDA_CHECK(slots < INT32_MAX && B * Hkv < 65535, TRIDA_ERR_ARG, "attn_canvas: grid too large");
  char* ws = static_cast<char*>(scratch);
  uint16_t* opart = reinterpret_cast<uint16_t*>(ws);
  float* mpart = reinterpret_cast<float*>(ws + align_up(slots * kMTX * D * 2, 256));
  float* lpart = reinterpret_cast<float*>(ws + align_up(slots * kMTX * D * 2, 256) + align_up(slots * kMTX * 4, 256));
  hipStream_t st = static_cast<hipStream_t>(stream);
  TRIDA_CHECK(!frag || B * T <= 48, TRIDA_ERR_ARG, "attn_canvas_frag: the fragment order holds at most 48 rows");
  AttnArgs a{q,           k_cache,         v_cache,          prefix_len, opart, mpart, lpart, (int)T, (int)Hq, (int)Hkv,
             (int)G,      (int)Lmax,       (int)S,           (int)QT,    mask_mode, (int)n_clean, scale * kLog2e, gate,
             gate_row_stride, gate_head_stride, out,         frag ? 1 : 0};
  const dim3 grid((unsigned)slots);
  switch (D) {
    case 64: hipLaunchKernelGGL(attn_partial_kernel<64>, grid, dim3(kNW * kWave), 0, st, a); break;
    case 128: hipLaunchKernelGGL(attn_partial_kernel<128>, grid, dim3(kNW * kWave), 0, st, a); break;
    default: hipLaunchKernelGGL(attn_partial_kernel<256>, grid, dim3(kNW * kWave), 0, st, a); break;
  }
  int rc = launch_status("attn_canvas/partial");
  if (rc || S == 1) return rc;  // one split: the partial kernel wrote the output
  CombineArgs c{opart, mpart, lpart, gate, out, (int)T, (int)Hq, (int)Hkv, (int)G, (int)D, (int)S, (int)QT,
                gate_row_stride, gate_head_stride, frag ? 1 : 0};
  if (S == 2 && !combine_general) {
    const dim3 cgrid((unsigned)cdiv(T * G, kC2T / (D / 4)), (unsigned)(B * Hkv));
    switch (D) {
      case 64: hipLaunchKernelGGL(attn_combine2_kernel<64>, cgrid, dim3(kC2T), 0, st, c); break;
      case 128: hipLaunchKernelGGL(attn_combine2_kernel<128>, cgrid, dim3(kC2T), 0, st, c); break;
      default: hipLaunchKernelGGL(attn_combine2_kernel<256>, cgrid, dim3(kC2T), 0, st, c); break;
    }
    return launch_status("attn_canvas/combine2");
  }
  const int64_t rows_per_block = kCT / (D / 4);
  const dim3 cgrid((unsigned)cdiv(T * G, rows_per_block), (unsigned)(B * Hkv));
  switch (D) {
    case 64: hipLaunchKernelGGL(attn_combine_kernel<64>, cgrid, dim3(kCT), 0, st, c); break;
    case 128: hipLaunchKernelGGL(attn_combine_kernel<128>, cgrid, dim3(kCT), 0, st, c); break;
    default: hipLaunchKernelGGL(attn_combine_kernel<256>, cgrid, dim3(kCT), 0, st, c); break;
  }
  return launch_status("attn_canvas/combine");
}
}  // namespace

extern "C" int trida_attn_set_combine_general(int on) {
  combine_general = on != 0;
  return TRIDA_OK;
}

extern "C" int trida_attn_canvas(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                 const int32_t* prefix_len, const uint16_t* gate, int64_t gate_row_stride,
                                 int64_t gate_head_stride, uint16_t* out, int64_t B, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                 int64_t Lmax, int mask_mode, int64_t n_clean, float scale, int64_t max_keys,
                                 int64_t splits, void* scratch, int64_t scratch_bytes, void* stream) {
  return attn_canvas_run(q, k_cache, v_cache, prefix_len, gate, gate_row_stride, gate_head_stride, out, false, B, T, Hq,
                         Hkv, D, Lmax, mask_mode, n_clean, scale, max_keys, splits, scratch, scratch_bytes, stream);
}

extern "C" int trida_attn_canvas_frag(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                      const int32_t* prefix_len, const uint16_t* gate, int64_t gate_row_stride,
                                      int64_t gate_head_stride, uint16_t* out_frag, int64_t B, int64_t T, int64_t Hq,
                                      int64_t Hkv, int64_t D, int64_t Lmax, int mask_mode, int64_t n_clean, float scale,
                                      int64_t max_keys, int64_t splits, void* scratch, int64_t scratch_bytes,
                                      void* stream) {
  return attn_canvas_run(q, k_cache, v_cache, prefix_len, gate, gate_row_stride, gate_head_stride, out_frag, true, B,
                         T, Hq, Hkv, D, Lmax, mask_mode, n_clean, scale, max_keys, splits, scratch, scratch_bytes,
                         stream);
}
