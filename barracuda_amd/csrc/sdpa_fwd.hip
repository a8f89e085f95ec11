// sdpa_fwd.hip -- fused scaled-dot-product attention forward for gfx950.
//
// Replaces the reference's three-pass attention (crates/barracuda/src/ops/
// attention/compute.rs:21-111: K6 shaders/math/attention_matmul_f64.wgsl
// writes the [B,H,Sq,Skv] scores, K7 activation/attention_softmax_f64.wgsl
// normalises them, K9 attention/attention_apply_f64.wgsl multiplies by V),
// its causal variant (ops/causal_attn/compute.rs:24-115 with K8, and the CPU
// ops/causal_attention.rs:52-134) and FlashAttention (ops/flash_attention.rs
// :96-145, K13).  Contract: o[b,h,i,:] = sum_j softmax_j(scale q_i . k_j) v_j,
// j <= i when causal.  The score matrix is never written to memory.
//
// Layout: per tensor a (batch, head, row) stride in elements with the head
// dimension contiguous; [B,H,S,D] row-major is the dense case.  K and V may
// have fewer heads than Q (grouped-query attention, ops/
// grouped_query_attention/compute.rs:27-121): query head h reads key/value
// head h / (H / Hkv).  Strided views also give multi-head attention its
// head split and concat for free (ops/mha/projections.rs:18-58 copy
// [B,S,H*D] <-> [B,H,S,D] through head_split_f64.wgsl / head_concat_f64.wgsl;
// here the kernel reads and writes the [B,S,H,D] projections in place).
//
// Head dimensions: D <= 128 run sdpa_fwd_kernel (below); 128 < D <= 256
// run sdpa_fwd16_kernel (16 queries per wavefront, further down); larger D
// take the chunked three-step path of sdpa_wide.hip.
//
// Design (FP32 MFMA for both products, v_mfma_f32_32x32x2_f32):
//   * A workgroup = 4 wavefronts = 128 queries of one (b,h); wavefront w owns
//     queries q0 + 32w .. +31, lane l's query is l % 32.  Key blocks of 32 are
//     streamed through LDS, double-buffered, one barrier per block; blocks are
//     loaded two ahead (the top of iteration t stores block t + 1 and issues
//     the loads of block t + 2), which took causal 1.14 -> 1.10 ms at
//     config 5: one block ahead, the compiler sank half of the loads down to
//     their LDS stores and every block waited out a load latency.
//   * Measured and not kept (config 5, same box, A/B): 512-thread
//     workgroups of 256 queries (half the K/V traffic per FLOP; -1% /
//     +2%); fragment reads pinned two chunks ahead; independent
//     accumulators for the QK^T and PV chains (no change: dependent MFMA
//     chains issue back to back); software-pipelining QK^T of block t + 1
//     against the softmax of block t with branch-free masking and rescale
//     (+2% / +4% time: the compiler kept the two phases apart and the
//     unconditional rescale added work).
//   * Scores are computed transposed, S^T = K Q^T (32 keys x 32 queries), so
//     each lane holds 16 scores of ITS query: the row max and row sum are
//     in-lane plus one exchange between the two lane halves.  The q operand
//     stays in registers for the whole kernel, pre-multiplied by
//     scale*log2(e) so the softmax uses exp2 directly.
//   * The PV product is computed as O^T += V^T P^T, whose B operand is
//     exactly the P values the lane already holds (value r of the S^T block
//     is key 8(r/4) + 4(l/32) + r%4), so P never leaves registers.  V is
//     stored transposed in LDS ([d][key]) so the A operand is one 128-bit
//     LDS read per four MFMAs; K is stored [key][d] for the same reason.
//   * Online softmax with a lazily moved reference max: exponentials are
//     taken against a per-query reference m_ref, which only moves (and O and
//     the running sum are only rescaled) when a block's max exceeds it by
//     more than 2^8.  Every term stays <= 256 and the final O / l is exact
//     algebra, so accuracy is unchanged while the rescale of the 64-value O
//     accumulator -- the costliest vector work per block -- almost never runs.
//   * Causal: key blocks past the workgroup's last query are not loaded;
//     blocks entirely above a wavefront's diagonal are skipped by that
//     wavefront; the diagonal block is masked per element.  Workgroups are
//     issued longest first across all heads (query block major); with
//     B*H % 8 == 0 every query block of a head then lands on one XCD.
//   * Non-causal: workgroups are issued head-major and remapped so that each
//     XCD (dispatch is round-robin over the 8 XCDs) runs a contiguous range
//     of heads, all query blocks of a head together.  The co-resident
//     workgroups of an XCD then cover 4 heads instead of 16, and each head's
//     K/V blocks are fetched into that XCD's L2 once for up to 16 readers:
//     at config 5, L2 misses 18.6 M -> 4.2 M and HBM fetch 2.2 -> 0.4 GB per
//     launch.  Query heads sharing a key/value head (grouped-query) are
//     adjacent, so they share it in the same L2.
//   * The max and sum exchanges between the two lane halves are
//     v_permlane32_swap (a VALU op) rather than an LDS-routed shuffle, which
//     sat on the path from the last QK^T MFMA to the first PV MFMA.
//     Together with the order above, against the previous kernel on one
//     box: non-causal 2.22 -> 2.20 ms, causal 1.11 -> 1.10, grouped-query
//     2.08 -> 2.06 (on another box the order alone: 2.23 -> 2.18).
//   * Measured and not kept: s_setprio 1 over each wave's MFMA phases
//     (non-causal 0-2% faster, causal 1-2% slower); head-major order for
//     causal too (1.10 -> 1.45 ms: a head's long query blocks then run
//     together, unbalanced); causal in groups of 4 heads per XCD, longest
//     first within a group (1.18 ms).
#include "bch_internal.h"

#include <math.h>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBKV = 32;  // keys per block
constexpr int kVLD = kBKV + 4;
constexpr float kLog2E = 1.44269504088896340736f;
constexpr float kLazy = 8.0f;  // log2 headroom before the reference max moves

// NT threads per workgroup: NT / 64 wavefronts of 32 queries each.
template <int DP, int NT>
struct SdpaCfg {
  static constexpr int BQ = NT / 2;                    // queries per workgroup
  static constexpr int KLD = DP + 4;
  static constexpr int KD4 = DP / 4;                   // float4 per K row
  static constexpr int K_TOT = kBKV * DP / 4;          // float4 of K per tile
  static constexpr int K_F4 = (K_TOT + NT - 1) / NT;    // float4 of K per thread
  static constexpr int V_BLK = kBKV * DP / 16;          // 4x4 V blocks per tile
  static constexpr int V_PER = (V_BLK + NT - 1) / NT;    // 4x4 V blocks per thread
  static constexpr int LDS_FLOATS = 2 * (kBKV * KLD + DP * kVLD);
  static_assert(K_F4 >= 1, "K tile must cover the workgroup");
};

// Staging registers for one key/value block, as vector values rather than
// float4 arrays: carried across the loop back-edge, the arrays were left in
// scratch memory.  Element 4f + e is component e of float4 number f.
template <int N>
using f32v = float __attribute__((ext_vector_type(N)));
template <int DP, int NT>
struct KvRegs {
  f32v<4 * SdpaCfg<DP, NT>::K_F4> k;
  f32v<16 * SdpaCfg<DP, NT>::V_PER> v;
};

// x combined with x from lane l ^ 32, the same value in both halves.
// v_permlane32_swap of (x, x) returns, per lane, {x[l & 31], x[(l & 31) + 32]}.
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float4 get4(const float* p) { return *reinterpret_cast<const float4*>(p); }

template <int DP, int NT, bool FULL>
__device__ __forceinline__ void load_k(const float* __restrict__ kh, long long ldk, int Skv, int D, int kb, int tid,
                                       KvRegs<DP, NT>& r) {
  using G = SdpaCfg<DP, NT>;
#pragma unroll
  for (int f = 0; f < G::K_F4; ++f) {
    const int idx0 = tid + f * NT;
    const int idx = (G::K_TOT % NT == 0 || idx0 < G::K_TOT) ? idx0 : 0;  // past the tile: reload float4 0 (unused)
    const int key = idx / G::KD4, d0 = (idx % G::KD4) * 4;
    const int gk = kb + key;
    float t[4];
    if (FULL) {
      const float4 x = get4(kh + gk * ldk + d0);
      t[0] = x.x; t[1] = x.y; t[2] = x.z; t[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = (gk < Skv && d0 + e < D) ? kh[gk * ldk + d0 + e] : 0.0f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) r.k[4 * f + e] = t[e];
  }
}

template <int DP, int NT, bool FULL>
__device__ __forceinline__ void load_v(const float* __restrict__ vh, long long ldv, int Skv, int D, int kb, int tid,
                                       KvRegs<DP, NT>& r) {
  using G = SdpaCfg<DP, NT>;
#pragma unroll
  for (int p = 0; p < G::V_PER; ++p) {
    const int idx = tid + p * NT;
    const int blk = idx < G::V_BLK ? idx : 0;  // threads past the tile reload block 0 (unused)
    const int kq = blk / G::KD4, dq = blk % G::KD4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int gk = kb + 4 * kq + e, d0 = 4 * dq;
      float t[4];
      if (FULL) {
        const float4 x = get4(vh + gk * ldv + d0);
        t[0] = x.x; t[1] = x.y; t[2] = x.z; t[3] = x.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) t[c] = (gk < Skv && d0 + c < D) ? vh[gk * ldv + d0 + c] : 0.0f;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) r.v[16 * p + 4 * e + c] = t[c];
    }
  }
}

template <int DP, int NT>
__device__ __forceinline__ void store_kv(float* __restrict__ ks, float* __restrict__ vt, int tid,
                                         const KvRegs<DP, NT>& r) {
  using G = SdpaCfg<DP, NT>;
#pragma unroll
  for (int f = 0; f < G::K_F4; ++f) {
    const int idx = tid + f * NT;
    if (G::K_TOT % NT == 0 || idx < G::K_TOT) {
      const int key = idx / G::KD4, d0 = (idx % G::KD4) * 4;
      *reinterpret_cast<float4*>(ks + key * G::KLD + d0) =
          make_float4(r.k[4 * f], r.k[4 * f + 1], r.k[4 * f + 2], r.k[4 * f + 3]);
    }
  }
#pragma unroll
  for (int p = 0; p < G::V_PER; ++p) {
    const int idx = tid + p * NT;
    if (G::V_BLK % NT == 0 || idx < G::V_BLK) {
      // transpose the 4(key) x 4(d) block: row d of Vt gets keys 4kq .. 4kq + 3
      const int kq = idx / G::KD4, dq = idx % G::KD4;
      float* base = vt + (4 * dq) * kVLD + 4 * kq;
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<float4*>(base + c * kVLD) =
            make_float4(r.v[16 * p + c], r.v[16 * p + 4 + c], r.v[16 * p + 8 + c], r.v[16 * p + 12 + c]);
    }
  }
}

template <int DP, bool FULL, int NT>
__global__ __launch_bounds__(NT, 2) void sdpa_fwd_kernel(
    int H, int group, int BH, int Sq, int Skv, int D, float qscale, int causal, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ o, bch::SdpaStrides st,
    int qblocks) {
  using G = SdpaCfg<DP, NT>;
  constexpr int KLD = G::KLD, kBQ = G::BQ;
  extern __shared__ float4 smem4[];
  float* smem = reinterpret_cast<float*>(smem4);
  float* Ks = smem;                        // [2][kBKV][KLD]
  float* Vt = smem + 2 * kBKV * KLD;       // [2][DP][kVLD]

  // causal: query-block major, all heads' longest query blocks first.
  // non-causal: head-major over an XCD-contiguous remap of the grid.
  int qi, bh;
  if (causal) {
    qi = blockIdx.x / BH;
    bh = blockIdx.x % BH;
  } else {
    const int nb = gridDim.x;
    int L = blockIdx.x;
    if ((nb & 7) == 0) L = (L & 7) * (nb >> 3) + (L >> 3);
    bh = L / qblocks;
    qi = L - bh * qblocks;
  }
  const int qb = causal ? qblocks - 1 - qi : qi;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 31, lh = lane >> 5;
  const int q0w = qb * kBQ + wave * 32;  // first query of this wavefront
  const int myq = q0w + li;

  const int bi = bh / H, hq = bh - bi * H, hk = hq / group;
  const float* qh = q + bi * st.q.batch + hq * st.q.head;
  const float* kh = k + bi * st.k.batch + hk * st.k.head;
  const float* vh = v + bi * st.v.batch + hk * st.v.head;
  float* oh = o + bi * st.o.batch + hq * st.o.head;

  // ---- q operand: qf[c] = q[myq][8c + 4lh .. +3] * scale * log2(e) ----
  float4 qf[DP / 8];
#pragma unroll
  for (int c = 0; c < DP / 8; ++c) {
    const int d0 = 8 * c + 4 * lh;
    float t[4];
    if (FULL) {
      const float4 x = *reinterpret_cast<const float4*>(qh + myq * st.q.row + d0);
      t[0] = x.x; t[1] = x.y; t[2] = x.z; t[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = (myq < Sq && d0 + e < D) ? qh[myq * st.q.row + d0 + e] : 0.0f;
    }
    qf[c] = make_float4(t[0] * qscale, t[1] * qscale, t[2] * qscale, t[3] * qscale);
  }

  f32x16 oacc[DP / 32];
#pragma unroll
  for (int b = 0; b < DP / 32; ++b)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[b][r] = 0.0f;
  float m_ref = -INFINITY, l_run = 0.0f;

  int kend = Skv;
  if (causal) kend = min(Skv, qb * kBQ + kBQ);
  const int nkb = (kend + kBKV - 1) / kBKV;

  // Key/value blocks are loaded two ahead: the top of iteration t stores
  // block t + 1 (loaded during iteration t - 1) into the buffer the previous
  // barrier released, then issues the loads of block t + 2.  With the loads
  // one block ahead and stored at the bottom, the compiler moved half of them
  // down to their stores, exposing a full load latency per block.
  // Blocks past the end are clamped to the last one (reloaded, never read).
  // (nkb >= 1: Skv >= 1 is validated, and a causal block row has >= 1 key)
  KvRegs<DP, NT> kv;
  load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, 0, tid, kv);
  load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, 0, tid, kv);
  store_kv<DP, NT>(Ks, Vt, tid, kv);
  load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, min(1, nkb - 1) * kBKV, tid, kv);
  load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, min(1, nkb - 1) * kBKV, tid, kv);
  __syncthreads();

  for (int t = 0; t < nkb; ++t) {
    const int cur = t & 1;
    const int kb = t * kBKV;
    store_kv<DP, NT>(Ks + (cur ^ 1) * kBKV * KLD, Vt + (cur ^ 1) * DP * kVLD, tid, kv);
    const int kbn = min(t + 2, nkb - 1) * kBKV;
    load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, kbn, tid, kv);
    load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, kbn, tid, kv);

    // wave-uniform: skip blocks fully above this wavefront's diagonal and
    // wavefronts whose queries are all past Sq
    const bool active = (q0w < Sq) && !(causal && kb > q0w + 31);
    if (active) {
      const float* ks = Ks + cur * kBKV * KLD + li * KLD + 4 * lh;
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < DP / 8; ++c) {
        const float4 kf = *reinterpret_cast<const float4*>(ks + 8 * c);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[c].x, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[c].y, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[c].z, s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[c].w, s, 0, 0, 0);
      }
      // value r: key kb + 8(r/4) + 4lh + r%4, query myq
      const bool need_mask = (!FULL && kb + kBKV > Skv) || (causal && kb + kBKV - 1 > q0w);
      if (need_mask) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (key >= Skv || (causal && key > myq)) s[r] = -INFINITY;
        }
      }
      float bm = s[0];
#pragma unroll
      for (int r = 1; r < 16; ++r) bm = fmaxf(bm, s[r]);
      bm = half_swap_max(bm);
      // move the reference max only when this block exceeds it by > 2^kLazy
      const bool move = bm > m_ref + kLazy;  // -inf reference: any finite block max moves it
      if (__any(move)) {
        const float m_new = move ? bm : m_ref;
        const float alpha = (m_ref == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
#pragma unroll
        for (int b = 0; b < DP / 32; ++b)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[b][r] *= alpha;
        m_ref = m_new;
      }
      const float m_use = (m_ref == -INFINITY) ? 0.0f : m_ref;
      float rs = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - m_use);
        rs += s[r];
      }
      rs = half_swap_sum(rs);
      l_run += rs;

      const float* vs = Vt + cur * DP * kVLD + li * kVLD + 4 * lh;
#pragma unroll
      for (int b = 0; b < DP / 32; ++b) {
#pragma unroll
        for (int a = 0; a < 4; ++a) {
          const float4 vf = *reinterpret_cast<const float4*>(vs + b * 32 * kVLD + 8 * a);
          oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.x, s[4 * a + 0], oacc[b], 0, 0, 0);
          oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.y, s[4 * a + 1], oacc[b], 0, 0, 0);
          oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.z, s[4 * a + 2], oacc[b], 0, 0, 0);
          oacc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.w, s[4 * a + 3], oacc[b], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: value r of block b is d = 32b + 8(r/4) + 4lh + r%4 ----
  if (myq < Sq) {
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int b = 0; b < DP / 32; ++b) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * b + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (FULL || d < D) oh[myq * st.o.row + d] = oacc[b][r] * inv;
      }
    }
  }
}

// ---- 128 < D <= 256: v_mfma_f32_16x16x4_f32, 16 queries per wavefront ----
// The 32x32 layout above keeps D/2 floats of q and D/2 of O per lane: at
// D = 256 that is 256 registers before staging and scores, one wavefront per
// SIMD, with the softmax of each block exposed on its SIMD.  Here a
// wavefront owns 16 queries, so q and O take D/4 floats each (64 + 64 at
// D = 256) and two wavefronts share each SIMD: 8 wavefronts = 128 queries
// per workgroup, the same K/V tile reuse and LDS layout as the 32x32 kernel
// (one workgroup per CU at 137 KB of LDS for D = 256).
//   S^T = K Q^T on 16 x 16 blocks: lane (g = l / 16, i = l % 16) supplies
//     K[key 16 sb + i][d] and q[query i][d] with d = 16 c + 4 g + e in step
//     (c, e), so one 128-bit LDS read of K and one register float4 of q feed
//     four MFMAs; value r of the result is key 16 sb + 4 g + r of query i.
//     A 32-key block is two such chains (sb = 0, 1): 8 scores per lane.
//   Row max and sum: in-lane over the 8, then across the four lanes
//     i, i + 16, i + 32, i + 48 of a query (v_permlane16_swap then
//     v_permlane32_swap; every lane of a query gets the same bits).
//   O^T += V^T P^T: step (sb, r) contracts key 16 sb + 4 g + r, whose P is
//     this lane's score r of chain sb; V^T comes from the transposed V tile
//     as one 128-bit read per four MFMAs.  Value r of O block db is
//     d = 16 db + 4 g + r of query i: the epilogue stores a float4.
// The online softmax (lazy reference max), causal skipping and masking and
// the workgroup order are those of sdpa_fwd_kernel.
// Measured at B=4, H=32, S=2048, D=256 (one box): 4.27 / 2.27 ms non-causal /
// causal (81.9% / 77.1% of FP32 MFMA peak), against 5.01 / 2.75 ms for
// sdpa_fwd_kernel at D = 256 (one wavefront per SIMD, accumulators in
// AGPRs).  D = 160 / 192 / 224: 75% / 77% / 79% non-causal.  For D <= 128
// this layout is slower than the 32x32 kernel (2.15 against 2.05 ms at
// config 5, 4 wavefronts per SIMD), so it starts above 128.
constexpr int kNT16 = 512;        // threads per workgroup: 8 wavefronts
constexpr int kBQ16 = kNT16 / 4;  // queries per workgroup (16 per wavefront)

typedef float f32x4v __attribute__((ext_vector_type(4)));

// x combined over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four lanes of one
// query), the same bits in all four: v_permlane16_swap of (x, x) returns
// {x[l & ~16], x[l | 16]} and v_permlane32_swap {x[l & ~32], x[l | 32]}.
__device__ __forceinline__ float quad_swap_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float quad_swap_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int DP, bool FULL>
__global__ __launch_bounds__(kNT16, 2) void sdpa_fwd16_kernel(
    int H, int group, int BH, int Sq, int Skv, int D, float qscale, int causal, const float* __restrict__ q,
    const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ o, bch::SdpaStrides st,
    int qblocks) {
  using G = SdpaCfg<DP, kNT16>;
  constexpr int KLD = G::KLD, NT = kNT16;
  extern __shared__ float4 smem4[];
  float* smem = reinterpret_cast<float*>(smem4);
  float* Ks = smem;                        // [2][kBKV][KLD]
  float* Vt = smem + 2 * kBKV * KLD;       // [2][DP][kVLD]

  int qi, bh;
  if (causal) {
    qi = blockIdx.x / BH;
    bh = blockIdx.x % BH;
  } else {
    const int nb = gridDim.x;
    int L = blockIdx.x;
    if ((nb & 7) == 0) L = (L & 7) * (nb >> 3) + (L >> 3);
    bh = L / qblocks;
    qi = L - bh * qblocks;
  }
  const int qb = causal ? qblocks - 1 - qi : qi;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int q0w = qb * kBQ16 + wave * 16;  // first query of this wavefront
  const int myq = q0w + li;

  const int bi = bh / H, hq = bh - bi * H, hk = hq / group;
  const float* qh = q + bi * st.q.batch + hq * st.q.head;
  const float* kh = k + bi * st.k.batch + hk * st.k.head;
  const float* vh = v + bi * st.v.batch + hk * st.v.head;
  float* oh = o + bi * st.o.batch + hq * st.o.head;

  // ---- q operand: qf[c] = q[myq][16c + 4lg .. +3] * scale * log2(e) ----
  float4 qf[DP / 16];
#pragma unroll
  for (int c = 0; c < DP / 16; ++c) {
    const int d0 = 16 * c + 4 * lg;
    float t[4];
    if (FULL) {
      const float4 x = *reinterpret_cast<const float4*>(qh + myq * st.q.row + d0);
      t[0] = x.x; t[1] = x.y; t[2] = x.z; t[3] = x.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = (myq < Sq && d0 + e < D) ? qh[myq * st.q.row + d0 + e] : 0.0f;
    }
    qf[c] = make_float4(t[0] * qscale, t[1] * qscale, t[2] * qscale, t[3] * qscale);
  }

  f32x4v oacc[DP / 16];
#pragma unroll
  for (int b = 0; b < DP / 16; ++b) oacc[b] = (f32x4v){0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY, l_run = 0.0f;

  int kend = Skv;
  if (causal) kend = min(Skv, qb * kBQ16 + kBQ16);
  const int nkb = (kend + kBKV - 1) / kBKV;

  KvRegs<DP, NT> kv;
  load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, 0, tid, kv);
  load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, 0, tid, kv);
  store_kv<DP, NT>(Ks, Vt, tid, kv);
  load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, min(1, nkb - 1) * kBKV, tid, kv);
  load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, min(1, nkb - 1) * kBKV, tid, kv);
  __syncthreads();

  for (int t = 0; t < nkb; ++t) {
    const int cur = t & 1;
    const int kb = t * kBKV;
    store_kv<DP, NT>(Ks + (cur ^ 1) * kBKV * KLD, Vt + (cur ^ 1) * DP * kVLD, tid, kv);
    const int kbn = min(t + 2, nkb - 1) * kBKV;
    load_k<DP, NT, FULL>(kh, st.k.row, Skv, D, kbn, tid, kv);
    load_v<DP, NT, FULL>(vh, st.v.row, Skv, D, kbn, tid, kv);

    const bool active = (q0w < Sq) && !(causal && kb > q0w + 15);
    if (active) {
      const float* ks = Ks + cur * kBKV * KLD + li * KLD + 4 * lg;
      f32x4v s[2];
      s[0] = s[1] = (f32x4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < DP / 16; ++c) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const float4 kf = *reinterpret_cast<const float4*>(ks + sb * 16 * KLD + 16 * c);
          s[sb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.x, qf[c].x, s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.y, qf[c].y, s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.z, qf[c].z, s[sb], 0, 0, 0);
          s[sb] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf.w, qf[c].w, s[sb], 0, 0, 0);
        }
      }
      // value r of chain sb: key kb + 16 sb + 4 lg + r, query myq
      const bool need_mask = (!FULL && kb + kBKV > Skv) || (causal && kb + kBKV - 1 > q0w);
      if (need_mask) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = kb + 16 * sb + 4 * lg + r;
            if (key >= Skv || (causal && key > myq)) s[sb][r] = -INFINITY;
          }
      }
      float bm = s[0][0];
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r) bm = fmaxf(bm, s[sb][r]);
      bm = quad_swap_max(bm);
      const bool move = bm > m_ref + kLazy;
      if (__any(move)) {
        const float m_new = move ? bm : m_ref;
        const float alpha = (m_ref == -INFINITY) ? 0.0f : __builtin_amdgcn_exp2f(m_ref - m_new);
        l_run *= alpha;
#pragma unroll
        for (int b = 0; b < DP / 16; ++b) oacc[b] *= alpha;
        m_ref = m_new;
      }
      const float m_use = (m_ref == -INFINITY) ? 0.0f : m_ref;
      float rs = 0.0f;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          s[sb][r] = __builtin_amdgcn_exp2f(s[sb][r] - m_use);
          rs += s[sb][r];
        }
      rs = quad_swap_sum(rs);
      l_run += rs;

      const float* vs = Vt + cur * DP * kVLD + li * kVLD + 4 * lg;
#pragma unroll
      for (int db = 0; db < DP / 16; ++db) {
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
          const float4 vf = *reinterpret_cast<const float4*>(vs + db * 16 * kVLD + 16 * sb);
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.x, s[sb][0], oacc[db], 0, 0, 0);
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.y, s[sb][1], oacc[db], 0, 0, 0);
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.z, s[sb][2], oacc[db], 0, 0, 0);
          oacc[db] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf.w, s[sb][3], oacc[db], 0, 0, 0);
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue: value r of block db is d = 16 db + 4 lg + r ----
  if (myq < Sq) {
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int db = 0; db < DP / 16; ++db) {
      const int d0 = 16 * db + 4 * lg;
      if (FULL) {
        *reinterpret_cast<float4*>(oh + myq * st.o.row + d0) =
            make_float4(oacc[db][0] * inv, oacc[db][1] * inv, oacc[db][2] * inv, oacc[db][3] * inv);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (d0 + r < D) oh[myq * st.o.row + d0 + r] = oacc[db][r] * inv;
      }
    }
  }
}

template <int DP, bool FULL>
hipError_t launch_dp16(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                       const float* q, const float* k, const float* v, float* o, const bch::SdpaStrides& st) {
  using G = SdpaCfg<DP, kNT16>;
  const int qblocks = (Sq + kBQ16 - 1) / kBQ16;
  const long long blocks = (long long)B * H * qblocks;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds = sizeof(float) * G::LDS_FLOATS;
  auto kern = sdpa_fwd16_kernel<DP, FULL>;
  hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(kern), (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(kNT16), lds, s, H, H / Hkv, B * H, Sq, Skv, D,
                     scale * kLog2E, causal, q, k, v, o, st, qblocks);
  return hipGetLastError();
}

template <int DP, bool FULL, int NT>
hipError_t launch_dp(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                     const float* q, const float* k, const float* v, float* o, const bch::SdpaStrides& st) {
  using G = SdpaCfg<DP, NT>;
  const int qblocks = (Sq + G::BQ - 1) / G::BQ;
  const long long blocks = (long long)B * H * qblocks;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  const size_t lds = sizeof(float) * G::LDS_FLOATS;
  auto kern = sdpa_fwd_kernel<DP, FULL, NT>;
  hipError_t e = bch::ensure_dynamic_lds(reinterpret_cast<const void*>(kern), (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(NT), lds, s, H, H / Hkv, B * H, Sq, Skv, D,
                     scale * kLog2E, causal, q, k, v, o, st, qblocks);
  return hipGetLastError();
}

bool aligned16(const float* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
bool mult4(const bch::SdpaLayout& l) { return l.batch % 4 == 0 && l.head % 4 == 0 && l.row % 4 == 0; }

template <int DP>
hipError_t launch_d(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                    const float* q, const float* k, const float* v, float* o, const bch::SdpaStrides& st) {
  constexpr int NT = 256;  // four wavefronts of 32 queries each
  // full tiles, 128-bit loads: every row start 16-byte aligned
  const bool full = D == DP && Sq % SdpaCfg<DP, NT>::BQ == 0 && Skv % kBKV == 0 && aligned16(q) && aligned16(k) &&
                    aligned16(v) && mult4(st.q) && mult4(st.k) && mult4(st.v);
  if (full) return launch_dp<DP, true, NT>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  return launch_dp<DP, false, NT>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
}

// 128 < D <= 256: the 16-query-per-wavefront kernel
template <int DP>
hipError_t launch_d16(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                      const float* q, const float* k, const float* v, float* o, const bch::SdpaStrides& st) {
  const bool full = D == DP && Sq % kBQ16 == 0 && Skv % kBKV == 0 && aligned16(q) && aligned16(k) && aligned16(v) &&
                    aligned16(o) && mult4(st.q) && mult4(st.k) && mult4(st.v) && mult4(st.o);
  if (full) return launch_dp16<DP, true>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  return launch_dp16<DP, false>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
}

}  // namespace

namespace bch {

hipError_t launch_sdpa_strided(hipStream_t s, int B, int H, int Hkv, int Sq, int Skv, int D, float scale,
                               int causal, const float* q, const float* k, const float* v, float* o,
                               const SdpaStrides& st) {
  if (Hkv < 1 || H % Hkv != 0) return hipErrorInvalidValue;
  if (D <= 32) return launch_d<32>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 64) return launch_d<64>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 128) return launch_d<128>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 160) return launch_d16<160>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 192) return launch_d16<192>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 224) return launch_d16<224>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  if (D <= 256) return launch_d16<256>(s, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, st);
  return hipErrorInvalidValue;
}

hipError_t launch_sdpa(hipStream_t s, int B, int H, int Sq, int Skv, int D, float scale, int causal,
                       const float* q, const float* k, const float* v, float* o) {
  SdpaStrides st;
  st.q = st.o = SdpaLayout{(long long)H * Sq * D, (long long)Sq * D, D};
  st.k = st.v = SdpaLayout{(long long)H * Skv * D, (long long)Skv * D, D};
  return launch_sdpa_strided(s, B, H, H, Sq, Skv, D, scale, causal, q, k, v, o, st);
}

}  // namespace bch
