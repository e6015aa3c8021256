// Forward of the dilution-attention operator (plain forward and chunked
// prefill share these kernels).
//
// Reference behaviour: dilution_attention_forward,
// /root/reference/src/dilution/kernels.py:328-455, whose row-parallel
// decomposition (K1 :137-198, block scan :251-264, K2 :267-315) this
// follows in its statistics and output passes; the kernels are written for
// gfx950 MFMA layouts:
//
//   prep       convert q/k to the MFMA operand type when needed; write V^T
//              (and K^T for pk) as contiguous (D, 32) tiles per 32 keys,
//              zero-padded to a multiple of 64 keys.
//   fwd_stats  row-parallel: one workgroup = 4 waves = 4 tiles of 32 query
//              rows, key tiles of 32 staged in LDS.  S^T = K Q^T puts one query
//              per lane: online row max and 2^-sum (log2 domain, lazily moved
//              offset), and optionally pk^T = K^T p^T on MFMA.
//   fwd_demand key-parallel: one wave per 32 keys walks the 32-row blocks in
//              causal order with the fp64 running column sum of p (plus any
//              incoming prefill demand) in a register, writing the demand that
//              enters every block (the carry checkpoints) and the totals
//              (committed_total, the decode accumulator).
//   fwd_out    row-parallel: S = Q K^T with keys in lanes: p, the in-tile
//              column scan on registers plus the checkpoint, share = p /
//              (demand + p + eps), row sums; the share tile is transposed by
//              one MFMA against an identity operand so that share @ V runs on
//              MFMA with queries in lanes.  out = (share @ V) / (rowsum + eps).
//
// Nothing T x T is stored: scratch is the (n, C/32, Tk) fp32 checkpoint array.
#pragma once

#include "dil_common.hpp"
#include "dil_internal.hpp"
#include "dil_tiles.hpp"
#include "dil_variant.hpp"

#include <type_traits>

namespace dil {

namespace {

struct FwdParams {
  const void* q;          // CT rows (n, C, D), slice stride q_sn
  int64_t q_sn;
  const void* k;          // CT rows (n, >= Tk, D), slice stride k_sn
  int64_t k_sn;
  const void* v;          // CT rows of V (n, >= Tk, D), slice stride v_sn: the key
  int64_t v_sn;           // pass parks V from them when set (else from vt)
  const void* vt;         // CT V^T, tile-major (Tk_pad rows per slice)
  const void* kt;         // CT K^T, tile-major, or null
  int64_t t_sn, tk_pad;
  int64_t C, Tk, q0, nb;
  int64_t n;              // slices
  int groups;             // 128-row groups per slice
  int kgroups;            // 128-key groups per slice
  float c;                // log2(e) / sqrt(D)
  float scale;            // 1 / sqrt(D)
  float shift, lshift;    // SHIFT of the expshift / sigshift bids and log2(SHIFT)
  float* out;
  int64_t o_sn;
  float* rmax;
  float* rden;
  float* ssum;
  float* carry;           // (n, nb, Tk)
  const float* demand_in;
  int64_t din_sn;
  float* total;
  int64_t tot_sn;
  float* pk;
  int lpt;                // dispatch longest first (xcd_work_item)
};

// ---------------------------------------------------------------------------
// Per-wave tile bounds.  A wave owns query rows [r0, r0 + 32) of the chunk
// (absolute rows qa0 = q0 + r0 ...).  Key tile kt (keys [32 kt, 32 kt + 32))
// needs no causal mask when kt < kfull and contributes nothing when
// kt >= kend.

struct WaveRows {
  int64_t r0, qa0;
  int kfull, kend;
  bool on;
};

__device__ __forceinline__ WaveRows wave_rows(const FwdParams& P, int g, int wave) {
  WaveRows w;
  w.r0 = (static_cast<int64_t>(g) * 4 + wave) * kTileQ;
  w.qa0 = P.q0 + w.r0;
  w.on = w.r0 < P.C;
  const int64_t qlast = min(w.qa0 + kTileQ - 1, P.q0 + P.C - 1);
  w.kend = w.on ? static_cast<int>(qlast / kTileK) + 1 : 0;
  w.kfull = w.on ? static_cast<int>((w.qa0 + 1) / kTileK) : 0;
  return w;
}

// Key tiles the workgroup (4 consecutive row tiles of group g) has to stage.
__device__ __forceinline__ int group_key_tiles(const FwdParams& P, int g) {
  const int64_t qlast = min(P.q0 + (static_cast<int64_t>(g) * 4 + 4) * kTileQ - 1, P.q0 + P.C - 1);
  return static_cast<int>(qlast / kTileK) + 1;
}

// Running maximum moves only when a tile exceeds it by this much (in units
// of the scaled log2 affinity), so the rescaling of the sums is rare; the
// terms 2^(a - m) then stay below 2^8.
constexpr float kLazyMax = 8.f;

// ---------------------------------------------------------------------------
// row statistics (+ pk) and per-32-row-block column sums of p

template <typename CT, int D, bool PK, int BID = BID_SOFTMAX>
__global__ __launch_bounds__(kThreads, 2) void fwd_stats(FwdParams P) {
  using T = Tiles<CT, D>;
  __shared__ __attribute__((aligned(16))) CT ktile[2][kTileK * T::kKStride];
  __shared__ __attribute__((aligned(16))) CT kttile[PK ? 2 : 1][PK ? D * T::kTStride : 1];
  // heavy (late) row groups first, over the whole chip when the slices do not
  // divide over the XCDs (spread)
  const WorkItem item = xcd_work_item(P.groups, P.n, true, P.lpt != 0, true);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int g = item.idx;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const WaveRows W = wave_rows(P, g, wave);
  const int nkt_wg = group_key_tiles(P, g);

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  const CT* ks = static_cast<const CT*>(P.k) + slice * P.k_sn;
  const CT* kts = PK ? static_cast<const CT*>(P.kt) + slice * P.t_sn : nullptr;

  // Q rows in natural order: the B operand of sweep 1 (lane <-> query) and the
  // A operand of sweep 2 (register rows <-> queries)
  RowFrag<CT, D> qf;
  const bool row_ok = W.r0 + l32 < P.C;
  if (row_ok) load_row_frag<CT, D>(qf, qs + (W.r0 + l32) * D + h * (D / 2));
  else zero_row_frag<CT, D>(qf);
  const int my_q = static_cast<int>(W.qa0) + l32;      // query of this lane in sweep 1

  if constexpr (!bid_normalized<BID>()) {
    // elementwise bids keep no row statistics (kernels_bid.py:338-349)
    if (h == 0 && row_ok) {
      P.rmax[slice * P.C + W.r0 + l32] = 0.f;
      P.rden[slice * P.C + W.r0 + l32] = BID == BID_EXPSHIFT ? P.shift : 1.f;
    }
    return;
  }

  KTileLoader<CT, D> kl;
  TTileLoader<CT, D> tl;

  // ---- sweep 1: S^T = K Q^T (lane <-> query, registers <-> keys) ----
  // softmax: m, the offset the sums are taken against (moves lazily), and mx,
  // the exact max; ratio bids: l = the row sum of the numerators, mn = the
  // row minimum of a (minshift)
  float m = -INFINITY, mx = -INFINITY, l0 = 0.f, l1 = 0.f, mn = INFINITY;
  floatx16 pka[PK ? kDTiles<D> : 1];
  if constexpr (PK) {
#pragma unroll
    for (int t = 0; t < kDTiles<D>; ++t) pka[t] = floatx16{};
  }
  const float thresh = kLazyMax / P.c;                 // in raw score units
  auto stats_step = [&](int kt, int buf, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    RowFrag<CT, D> kf;
    lds_row_frag<CT, D>(kf, ktile[buf], rho(l32), h);
    const floatx16 acc = mma_rows<CT, D>(kf, qf, floatx16{});
    float a[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = acc[i];
    if constexpr (bid_ratio<BID>()) {
      // numerators f(a) and Jacobian numerators u(a) on the causal window
      const int dq = kt * kTileK + 8 * h - my_q;
      float e[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const bool ok = !DIAG || 16 * (i >> 3) + (i & 7) + dq <= 0;
        const float av = a[i] * P.scale;
        const float f = ok ? bid_f<BID>(av) : 0.f;
        if (i & 1) l1 += f;
        else l0 += f;
        if constexpr (BID == BID_MINSHIFT) mn = ok ? fminf(mn, av) : mn;
        e[i] = ok ? bid_u<BID>(av) : 0.f;
      }
      if constexpr (PK) {
#pragma unroll
        for (int s = 0; s < kTileK / Mma<CT>::kStep; ++s) {
          const auto bfr = acc_frag<CT>(e, s);
#pragma unroll
          for (int t = 0; t < kDTiles<D>; ++t)
            pka[t] = Mma<CT>::mma(lds_t_frag<CT, D>(kttile[buf], 32 * t + l32, h, s), bfr, pka[t]);
        }
      }
      return;
    }
    if constexpr (DIAG) {
      const int dq = kt * kTileK + 8 * h - my_q;       // key - query for register i: perm_row(i, 0) + dq
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (16 * (i >> 3) + (i & 7) + dq > 0) a[i] = -INFINITY;
    }
    float tmax = fmaxf(fmaxf(a[0], a[1]), a[2]);
#pragma unroll
    for (int i = 3; i < 15; i += 2) tmax = fmaxf(fmaxf(tmax, a[i]), a[i + 1]);
    tmax = fmaxf(tmax, a[15]);
    const HalfPair tp = halves(tmax);                  // one running max per query (both halves)
    tmax = fmaxf(tp.lo, tp.hi);
    mx = fmaxf(mx, tmax);
    const bool take = tmax > m + thresh;
    if (__any(take)) {
      const float mnew = take ? tmax : m;
      const float alpha = take ? (m == -INFINITY ? 0.f : fast_exp2((m - mnew) * P.c)) : 1.f;
      l0 *= alpha;
      l1 *= alpha;
      if constexpr (PK) {
#pragma unroll
        for (int t = 0; t < kDTiles<D>; ++t) pka[t] *= alpha;
      }
      m = mnew;
    }
    const float mc = m * P.c;
    float e[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) e[i] = fast_exp2(fmaf(a[i], P.c, -mc));
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      l0 += e[i];
      l1 += e[i + 1];
    }
    if constexpr (PK) {
#pragma unroll
      for (int s = 0; s < kTileK / Mma<CT>::kStep; ++s) {
        const auto bfr = acc_frag<CT>(e, s);
#pragma unroll
        for (int t = 0; t < kDTiles<D>; ++t)
          pka[t] = Mma<CT>::mma(lds_t_frag<CT, D>(kttile[buf], 32 * t + l32, h, s), bfr, pka[t]);
      }
    }
  };

  kl.load(ks, 0, P.Tk);
  if constexpr (PK) tl.load(kts, 0);
  kl.store(ktile[0]);
  if constexpr (PK) tl.store(kttile[0]);
  __syncthreads();
  auto iter = [&](int kt, int buf) __attribute__((always_inline)) {
    if (kt + 1 < nkt_wg) {
      const int64_t key0n = static_cast<int64_t>(kt + 1) * kTileK;
      kl.load(ks, key0n, P.Tk);
      if constexpr (PK) tl.load(kts, key0n);
    }
    if (kt < W.kfull) stats_step(kt, buf, std::false_type{});
    else if (kt < W.kend) stats_step(kt, buf, std::true_type{});
    if (kt + 1 < nkt_wg) {
      kl.store(ktile[buf ^ 1]);
      if constexpr (PK) tl.store(kttile[buf ^ 1]);
    }
    sync_lds();
  };
  double_buffered<true>(0, nkt_wg, iter);
  const HalfPair lp = halves(l0 + l1);                 // the halves share m
  float ltot, rmax_v, pk_f;
  if constexpr (bid_ratio<BID>()) {
    // R = sum of the numerators; minshift: sum(a - min) = sum(a) - window * min
    ltot = lp.lo + lp.hi;
    rmax_v = 0.f;
    if constexpr (BID == BID_MINSHIFT) {
      const HalfPair mp = halves(mn);
      rmax_v = fminf(mp.lo, mp.hi);                    // the rmax buffer holds the row minimum
      ltot = fmaxf(ltot - static_cast<float>(my_q + 1) * rmax_v, 0.f);
    }
    pk_f = ltot > 0.f ? P.scale / ltot : 0.f;          // jac = u / R (0 on an empty row)
  } else {
    // re-reference the sum to the exact row maximum: p = 2^(a c - rmax) / rden
    ltot = (lp.lo + lp.hi) * fast_exp2((m - mx) * P.c);
    rmax_v = mx * P.c;
    pk_f = P.scale / (lp.lo + lp.hi);                  // pk was accumulated against m
  }
  if (h == 0 && row_ok) {
    P.rmax[slice * P.C + W.r0 + l32] = rmax_v;
    P.rden[slice * P.C + W.r0 + l32] = ltot;
  }
  if constexpr (PK) {
    if (row_ok) {
      const float f = pk_f;
      float* dst = P.pk + (slice * P.C + W.r0 + l32) * D;
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * t + acc_row(i, h) < D) dst[32 * t + acc_row(i, h)] = pka[t][i] * f;
    }
  }
}

// ---------------------------------------------------------------------------
// demand checkpoints: key-parallel walk over the chunk's 32-row blocks
//
// One wave per 32-key tile (lane <-> key).  Walking the row blocks in causal
// order it carries each key's demand -- the incoming demand of rows before the
// chunk plus the column sums of p over the chunk rows seen so far -- in an
// fp64 register, stores it as the checkpoint of every block (the demand
// entering the block) and finally as the key's total.

template <typename CT, int D, int BID = BID_SOFTMAX>
__global__ __launch_bounds__(kThreads, (sizeof(CT) == 2 && D <= 64) ? 4 : 2) void fwd_demand(FwdParams P) {
  using T = Tiles<CT, D>;
  constexpr int kRP = BID == BID_SOFTMAX ? 1 : 2;                  // per-row parameters
  __shared__ __attribute__((aligned(16))) CT q_s[2][kTileQ * T::kKStride];
  // (r0, r1) of the block's rows, then padding: every thread of the stash writes
  __shared__ __attribute__((aligned(16))) float st_s[2][kRP][kThreads];

  const WorkItem item = xcd_work_item(P.kgroups, P.n, false, P.lpt != 0);   // early keys (long walks) first
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int kb = item.idx * 4 + wave;
  const int64_t key0 = static_cast<int64_t>(kb) * kTileK;
  const int64_t key = key0 + l32;
  const bool key_ok = key < P.Tk;

  // Block b holds chunk rows [32 b, 32 b + 32) = absolute rows q0 + 32 b + [0, 32).
  // A key tile meets block b when the block's last row reaches its first key;
  // it needs no mask once the block's first row is past its last key.
  auto first_block = [&](int64_t k0) -> int64_t {
    const int64_t t = k0 - P.q0 - (kTileQ - 1);
    return t > 0 ? (t + kTileQ - 1) / kTileQ : 0;
  };
  const int64_t b_wg = first_block(static_cast<int64_t>(item.idx) * 4 * kTileK);
  const int64_t b_w = first_block(key0);
  const int64_t nb = P.nb;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  const float* rmax = P.rmax + slice * P.C;
  const float* rden = P.rden + slice * P.C;

  RowFrag<CT, D> kf;
  if (key_ok) load_row_frag<CT, D>(kf, static_cast<const CT*>(P.k) + slice * P.k_sn + key * D + h * (D / 2));
  else zero_row_frag<CT, D>(kf);

  double run = (P.demand_in != nullptr && key < P.q0 && key_ok)
                   ? static_cast<double>(P.demand_in[slice * P.din_sn + key]) : 0.0;
  float* ccol = P.carry + slice * nb * P.Tk + key;

  KTileLoader<CT, D> ql;
  float rmax_r = 0.f, rden_r = 1.f;
  bool row_ok = false;
  int64_t it_row0 = 0;                       // first chunk row of the fetched block
  auto fetch = [&](int64_t b) {
    it_row0 = b * kTileQ;
    ql.load(qs, b * kTileQ, P.C);
    const int64_t r = b * kTileQ + (threadIdx.x & (kTileQ - 1));
    row_ok = r < P.C;
    rmax_r = rmax[min(r, P.C - 1)];
    rden_r = rden[min(r, P.C - 1)];
  };
  auto stash = [&](int buf) {
    ql.store(q_s[buf]);
    // threads past the block's 32 rows write padding (no exec-masked branch
    // around the wait for the loaded statistics)
    if constexpr (BID == BID_SOFTMAX) {
      st_s[buf][0][threadIdx.x] = row_ok ? rmax_r + __log2f(rden_r) : INFINITY;
    } else {
      float r0, r1;
      const float window = static_cast<float>(P.q0 + (it_row0 + (threadIdx.x & (kTileQ - 1))) + 1);
      bid_row_params<BID>(rmax_r, rden_r, window, row_ok, r0, r1);
      st_s[buf][0][threadIdx.x] = r0;
      st_s[buf][1][threadIdx.x] = r1;
    }
  };

  auto step = [&](int64_t b, int buf, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    RowFrag<CT, D> qf;
    lds_row_frag<CT, D>(qf, q_s[buf], l32, h);
    const floatx16 acc = mma_rows<CT, D>(qf, kf, floatx16{});   // register i <-> row acc_row(i, h)
    float p[16];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const floatx4 r0 = *reinterpret_cast<const floatx4*>(&st_s[buf][0][8 * u + 4 * h]);
      if constexpr (BID == BID_SOFTMAX) {
#pragma unroll
        for (int e = 0; e < 4; ++e) p[4 * u + e] = fast_exp2(fmaf(acc[4 * u + e], P.c, -r0[e]));
      } else {
        const floatx4 r1 = *reinterpret_cast<const floatx4*>(&st_s[buf][kRP - 1][8 * u + 4 * h]);
#pragma unroll
        for (int e = 0; e < 4; ++e) p[4 * u + e] = bid_p<BID>(acc[4 * u + e], P.c, P.scale, r0[e], r1[e], P.lshift);
      }
    }
    if constexpr (DIAG) {
      // key - row for register i: dq - (8 (i >> 2) + (i & 3))
      const int dq = static_cast<int>(key - P.q0 - b * kTileQ) - 4 * h;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dq > 8 * (i >> 2) + (i & 3)) p[i] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) p[i] += p[i + 8];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] += p[i + 4];
    const HalfPair cp = halves((p[0] + p[1]) + (p[2] + p[3]));
    run += static_cast<double>(cp.lo + cp.hi);
  };

  // Blocks that end before this wave's first key never see it: their
  // checkpoints for these keys (the future triangle) are left unwritten, as
  // the reference leaves them (kernels.py:353-354), and no kernel reads them.
  if (b_wg < nb) {
    fetch(b_wg);
    stash(0);
  }
  __syncthreads();
  // vmcnt counts stores as well as loads: the stash is unconditional (the
  // last iteration stashes into the idle buffer) and the checkpoint is stored
  // after it, so that the wait for the fetched block never waits for a store
  auto iter = [&](int64_t b, int buf) __attribute__((always_inline)) {
    fetch(min(b + 1, nb - 1));                  // the last step reloads its own block, unused
    // wave-uniform condition: every lane must feed the MFMAs of the step
    const bool on = b >= b_w && key0 < P.Tk;
    const float entering = static_cast<float>(run);   // demand entering block b
    if (on) {
      const int64_t first_row = P.q0 + b * kTileQ;
      if (key0 + kTileK - 1 <= first_row) step(b, buf, std::false_type{});
      else step(b, buf, std::true_type{});
    }
    stash(buf ^ 1);
    if (on && h == 0 && key_ok) ccol[b * P.Tk] = entering;
    sync_lds();
  };
  double_buffered<true>(b_wg, nb, iter);
  if (key_ok && h == 0) P.total[slice * P.tot_sn + key] = static_cast<float>(run);
}

// ---------------------------------------------------------------------------
// output pass

template <typename CT, int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
__global__ __launch_bounds__(kThreads, 2) void fwd_out(FwdParams P) {
  using T = Tiles<CT, D>;
  constexpr int kRP = BID == BID_SOFTMAX ? 1 : 2;                  // per-row parameters
  // a stage holds two consecutive key tiles; two stages double-buffer them
  __shared__ __attribute__((aligned(16))) CT ktile[2][2][kTileK * T::kKStride];
  __shared__ __attribute__((aligned(16))) CT vttile[2][2][D * T::kTStride];
  __shared__ __attribute__((aligned(16))) float lse_s[4][kRP][kTileQ];
  __shared__ float ssum_s[4][kTileQ];
  __shared__ float cs_s[2][4][2 * kTileK];             // demand checkpoints per stage and wave

  const WorkItem item = xcd_work_item(P.groups, P.n, true, P.lpt != 0);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int g = item.idx;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const float hf = static_cast<float>(h);
  const WaveRows W = wave_rows(P, g, wave);
  const int nkt_wg = group_key_tiles(P, g);
  const int nst = (nkt_wg + 1) / 2;                    // stages of two key tiles

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  const CT* ks = static_cast<const CT*>(P.k) + slice * P.k_sn;
  const CT* vts = static_cast<const CT*>(P.vt) + slice * P.t_sn;

  // Q rows in QS order: accumulator register i of half h <-> row 16 h + i
  RowFrag<CT, D> qf;
  const int64_t my_row = W.r0 + qsig(l32);
  if (my_row < P.C) load_row_frag<CT, D>(qf, qs + my_row * D + h * (D / 2));
  else zero_row_frag<CT, D>(qf);

  // log2-sum-exp of this wave's rows (the per-row bid parameters of the
  // variants), read from LDS at every step (keeps registers for occupancy)
  if (h == 0) {
    const int64_t r = W.r0 + l32;
    const int64_t rc = min(r, P.C - 1);
    if constexpr (BID == BID_SOFTMAX) {
      lse_s[wave][0][l32] = (r < P.C) ? P.rmax[slice * P.C + r] + __log2f(P.rden[slice * P.C + r]) : INFINITY;
    } else {
      float r0, r1;
      bid_row_params<BID>(P.rmax[slice * P.C + rc], P.rden[slice * P.C + rc],
                          static_cast<float>(P.q0 + r + 1), r < P.C, r0, r1);
      lse_s[wave][0][l32] = r0;
      lse_s[wave][kRP - 1][l32] = r1;
    }
  }
  constexpr int kSteps = kTileK / Mma<CT>::kStep;
  typename Mma<CT>::frag ident[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) ident[s] = ident_qs<CT>(l32, h, s);
  floatx16 o[kDTiles<D>];
#pragma unroll
  for (int t = 0; t < kDTiles<D>; ++t) o[t] = floatx16{};
  // row sums of the shares: each lane adds the transposed shares of its row
  // (row l32, the keys of its half) on the VALU -- the values that multiply V
  float rsum = 0.f;

  // The demand checkpoints of a stage (each wave's rows, the stage's 64 keys)
  // are staged through LDS with the tiles: thread t loads the one of wave
  // t >> 6, key 32 * ((t >> 5) & 1) + (t & 31) of the stage.
  const int cw = threadIdx.x >> 6, cj = threadIdx.x & 63;
  const int64_t c_rb = min(static_cast<int64_t>(g) * 4 + cw, P.nb - 1);
  const float* c_row = P.carry + (slice * P.nb + c_rb) * P.Tk;
  // bf16 up to head_dim 64: the tile fetch runs two stages ahead into two
  // register sets (picked by the stage's parity, a constant in the unrolled
  // loop), because one stage of compute did not always cover the K/V load
  // latency (fwd_out -1.5% at B1 H16 T16384).  The other forms keep one set
  // (no registers to spare: fp32 and split operands would spill).
  constexpr bool kPf2 = std::is_same_v<CT, __bf16> && D <= 64;
  constexpr int kSets = kPf2 ? 2 : 1;
  float cr[kSets] = {};
  bool cr_ok[kSets] = {};

  // N consecutive key tiles kt0 .. kt0 + N - 1 of stage buffer `buf`, their
  // phases interleaved so that one tile's MFMAs overlap the other's VALU work
  auto out_tiles = [&](auto n_tag, auto diag_tag, int kt0, int slot0, int buf) {
    constexpr int N = decltype(n_tag)::value;
    constexpr bool DIAG = decltype(diag_tag)::value;
    float cin[N];
#pragma unroll
    for (int n = 0; n < N; ++n) cin[n] = cs_s[buf][wave][(slot0 + n) * kTileK + rho(l32)];
    floatx16 acc[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      RowFrag<CT, D> kf;
      lds_row_frag<CT, D>(kf, ktile[buf][slot0 + n], rho(l32), h);
      acc[n] = mma_rows<CT, D>(qf, kf, floatx16{});
    }
    float lse[16], rb1[16];
    {
      const floatx4* lp = reinterpret_cast<const floatx4*>(&lse_s[wave][0][16 * h]);
      const floatx4* lq = reinterpret_cast<const floatx4*>(&lse_s[wave][kRP - 1][16 * h]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const floatx4 v = lp[u];
        lse[4 * u] = v[0]; lse[4 * u + 1] = v[1]; lse[4 * u + 2] = v[2]; lse[4 * u + 3] = v[3];
        if constexpr (BID != BID_SOFTMAX) {
          const floatx4 w = lq[u];
          rb1[4 * u] = w[0]; rb1[4 * u + 1] = w[1]; rb1[4 * u + 2] = w[2]; rb1[4 * u + 3] = w[3];
        }
      }
    }
    float p[N][16], x[N][16];
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        if constexpr (BID == BID_SOFTMAX) p[n][i] = fast_exp2(fmaf(acc[n][i], P.c, -lse[i]));
        else p[n][i] = bid_p<BID>(acc[n][i], P.c, P.scale, lse[i], rb1[i], P.lshift);
      }
    if constexpr (DIAG) {
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const int dk = (kt0 + n) * kTileK + rho(l32) - static_cast<int>(W.qa0) - 16 * h;   // key - query(i) = dk - i
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (dk > i) p[n][i] = 0.f;
      }
    }
    if constexpr (SHARE != SHARE_NONE) {
#pragma unroll
      for (int n = 0; n < N; ++n) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[n][i] = p[n][i];
        if constexpr (SHARE == SHARE_EXCL) scan_excl_qs(x[n], cin[n] + kEps, hf);   // demand + eps
        else scan_incl_qs(x[n], cin[n] + kEps, hf);                                // demand + p + eps
      }
#pragma unroll
      for (int n = 0; n < N; ++n)
#pragma unroll
        for (int i = 0; i < 16; ++i) p[n][i] *= fast_rcp(x[n][i]);                 // share
    }
    // transpose each share tile: queries in lanes, keys (natural order) in registers
    floatx16 xt[N];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      xt[n] = floatx16{};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) xt[n] = Mma<CT>::mma_bexact(acc_frag<CT>(p[n], s), ident[s], xt[n]);
    }
#pragma unroll
    for (int n = 0; n < N; ++n) {
      float xv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xv[i] = xt[n][i];
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const auto af = acc_frag<CT>(xv, s);
#pragma unroll
        for (int t = 0; t < kDTiles<D>; ++t)
          o[t] = Mma<CT>::mma(af, lds_t_frag<CT, D>(vttile[buf][slot0 + n], 32 * t + l32, h, s), o[t]);
      }
      rsum += sum16(xv);
    }
  };

  KTileLoader<CT, D, false, kLoadClamp> kl[kSets][2];  // clamped global loads: measured faster here
  TTileLoader<CT, D, kLoadClamp> vl[kSets][2];
  auto fetch = [&](int st, int set) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      const int64_t key0 = static_cast<int64_t>(2 * st + n) * kTileK;
      kl[set][n].load(ks, key0, P.Tk);
      vl[set][n].load(vts, key0);
    }
    const int64_t key = static_cast<int64_t>(st) * 2 * kTileK + cj;
    cr_ok[set] = key < P.Tk;
    cr[set] = c_row[min(key, P.Tk - 1)];
  };
  auto stash = [&](int buf, int set) {
#pragma unroll
    for (int n = 0; n < 2; ++n) {
      kl[set][n].store(ktile[buf][n]);
      vl[set][n].store(vttile[buf][n]);
    }
    cs_s[buf][cw][cj] = cr_ok[set] ? cr[set] : 0.f;
  };
  fetch(0, 0);
  if constexpr (kPf2) fetch(min(1, nst - 1), 1);
  stash(0, 0);
  __syncthreads();
  // stage st + 1 sits in register set (st + 1) & 1 = buf ^ 1 (two-stage
  // prefetch) when its stash comes; the set just stashed takes stage st + 2
  auto iter = [&](int st, int buf) __attribute__((always_inline)) {
    const int kt0 = 2 * st;
    // the last stages reload the final one, unused
    if constexpr (kPf2) fetch(min(st + 2, nst - 1), buf);
    else fetch(min(st + 1, nst - 1), 0);
    if (kt0 + 1 < W.kfull) {
      out_tiles(std::integral_constant<int, 2>{}, std::false_type{}, kt0, 0, buf);
    } else {
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        if (kt0 + n < W.kfull)
          out_tiles(std::integral_constant<int, 1>{}, std::false_type{}, kt0 + n, n, buf);
        else if (kt0 + n < W.kend)
          out_tiles(std::integral_constant<int, 1>{}, std::true_type{}, kt0 + n, n, buf);
      }
    }
    if (st + 1 < nst) stash(buf ^ 1, kPf2 ? buf ^ 1 : 0);
    sync_lds();
  };
  // unrolled by two up to head_dim 64, which also makes buf (and the register
  // set) a constant in each copy; head_dim 128 has no registers to spare
  double_buffered<(D <= 64)>(0, nst, iter);

  // row sums: the two halves of row l32
  const HalfPair rp = halves(rsum);
  if (h == 0) ssum_s[wave][l32] = rp.lo + rp.hi;
  __syncthreads();
  if (h == 0 && W.r0 + l32 < P.C) P.ssum[slice * P.C + W.r0 + l32] = ssum_s[wave][l32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = acc_row(i, h);
    if (W.r0 + row < P.C) {
      const float inv = 1.f / (ssum_s[wave][row] + kEps);
      float* dst = P.out + slice * P.o_sn + (W.r0 + row) * D;
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
        if (32 * t + l32 < D) dst[32 * t + l32] = o[t][i] * inv;
    }
  }
}
// ---------------------------------------------------------------------------
// key-parallel output pass (bf16 operands, head_dim 64: the training forward
// and prefill chunks that start at a multiple of the group's keys)
//
// fwd_demand's walk, widened to KW waves = 32 KW keys per workgroup and
// forming the output in the same walk, so the scores, exp2 and demand scan
// run once after the statistics instead of twice.  A group's keys before the
// chunk start from the carried demand and meet every row tile of the chunk;
// the others start at their diagonal tile.  Per 32-row tile every wave (32
// keys, lane <-> key, rows in the query-split layout):
//   * p = 2^(a c - lse), masked on the diagonal tile;
//   * the demand entering the tile is the wave's running fp64 column sum
//     (stored as the tile's checkpoint for the backward); an in-register scan
//     gives demand + p + eps, the share p / (demand + p + eps), and the
//     running sum advances by the tile's column total;
//   * the share tile is transposed with an identity MFMA (rows in lanes) and
//     staged in LDS as bf16; its row sums (the normaliser's partial, over the
//     same bf16 values that multiply V) are added on the VALU.
// After the next tile's stash 8 waves form the tile's share V over the
// group's keys, one 16 x 16 output block each (v_mfma_f32_16x16x32_bf16, V
// parked in LDS), stored as one bf16 [64 x 32] partial (part_block_off) per (key group,
// tile) with the fp32 row sums beside it, compactly (ChunkGroups).
// fwd_out_reduce sums the partials of every key group in a fixed order and
// normalises.  With 16 waves (512 keys) a CU holds one workgroup (148 KB of
// LDS) and there are half the partials of 8 waves.

template <int D, int KW>
__global__ __launch_bounds__(64 * KW, 16 / KW) void fwd_keyout(FwdParams P, __bf16* __restrict__ op,
                                                               float* __restrict__ rp, int64_t ntiles) {
  static_assert(D == 64, "the key-parallel output pass is built for head_dim 64");
  static_assert(KW == 8 || KW == 16, "key groups of 256 or 512 keys");
  using CT = __bf16;
  using TL = Tiles<CT, D>;
  using KG = KeyGroups<KW>;
  __shared__ __attribute__((aligned(16))) CT q_s[2][kTileQ * TL::kKStride];
  __shared__ __attribute__((aligned(16))) float st_s[2][kTileQ];          // lse of the tile's rows
  __shared__ __attribute__((aligned(16))) CT sh_s[2][kTileQ * KG::kStride];  // shares, [row][key]
  __shared__ float rs_s[2][KW][kTileQ];                                    // row sums per wave
  // B operand of the share V product: V of the group's keys, per d quarter
  // and key step (32 keys), lane-minor
  __shared__ __attribute__((aligned(16))) bf16x8 vpark[D / 16][KW][64];
  __shared__ __attribute__((aligned(16))) bf16x8 id_park[2][64];          // transpose identity

  // early keys (long walks) first; a walk reads one row tile per step, so
  // balance across the XCDs matters more than L2 sharing (spread)
  const WorkItem item = xcd_work_item(P.kgroups, P.n, false, P.lpt != 0, true);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const float hf = static_cast<float>(h);
  const int kg = item.idx;
  const int kb0 = kg * KW;                       // first key tile of the group
  const int kb = kb0 + wave;                     // key tile of this wave
  const int64_t T = P.Tk;                        // keys [0, q0 + C)
  const int64_t C = P.C;                         // chunk rows [q0, q0 + C)
  const int q0t = static_cast<int>(P.q0 / kTileQ);   // global row tile of chunk row tile 0
  const ChunkGroups<KW> cg{(C + kTileQ - 1) / kTileQ, P.q0 / KG::kKeys};
  const int nq = static_cast<int>(cg.nq);
  const int rt0 = static_cast<int>(cg.first(kg));    // the group's first chunk row tile
  const int64_t key = static_cast<int64_t>(kb) * kTileK + l32;
  const bool key_ok = key < T;
  const bool active = static_cast<int64_t>(kb) * kTileK < T;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  RowFrag<CT, D> kf;
  if (key_ok) load_row_frag<CT, D>(kf, static_cast<const CT*>(P.k) + slice * P.k_sn + key * D + h * (D / 2));
  else zero_row_frag<CT, D>(kf);
  // the parked V fragments: fragment (d quarter u, key step w, lane) holds
  // V[32 (kb0 + w) + 8 (lane >> 4) + t][16 u + (lane & 15)], t = 0..7, zero
  // past the last key.  From the bf16 rows of V (no transposed copy to
  // write): chunk i of the group's rows (key i / 8, head dims 8 (i % 8) +
  // [0, 8)) is loaded whole, and its 8 values are written to their fragments
  // one by one.  Else 16 contiguous bytes of the tile-major V^T copy per
  // fragment.  Loaded here, written to LDS once the first row tile's fetch is
  // in flight too, so the walk starts after one memory wait instead of two.
  constexpr int kVChunks = KG::kKeys * D / 8 / KG::kThreads;     // 16-byte row chunks per thread
  bf16x8 vfr[kVChunks];
  static_assert(kVChunks == D / 16, "one register set serves both parking forms");
  if (P.v != nullptr) {
    const int64_t first = static_cast<int64_t>(kb0) * kTileK;            // the group's first key
    const CT* vs = static_cast<const CT*>(P.v) + slice * P.v_sn + first * D;
    const auto rs = make_rsrc(vs, (T - first) * D * static_cast<int64_t>(sizeof(CT)));
#pragma unroll
    for (int c = 0; c < kVChunks; ++c)
      vfr[c] = buffer_load16<bf16x8>(rs, static_cast<uint32_t>((threadIdx.x + c * KG::kThreads) * 16), 0);
  } else {
    const CT* vts = static_cast<const CT*>(P.vt) + slice * P.t_sn;
    const int64_t first = static_cast<int64_t>(kb0) * kTileK * D;
    const auto rs = make_rsrc(vts + first, (P.t_sn - first) * static_cast<int64_t>(sizeof(CT)));
#pragma unroll
    for (int u = 0; u < D / 16; ++u) {
      const int d = 16 * u + (lane & 15);
      const uint32_t off = static_cast<uint32_t>(((wave * D + d) * kTileK + 8 * (lane >> 4)) * sizeof(CT));
      vfr[u] = buffer_load16<bf16x8>(rs, off, 0);
    }
  }
  // demand entering the current tile (this lane's key): the carried demand of
  // the rows before the chunk for its earlier keys
  double run = (P.demand_in != nullptr && key < P.q0 && key_ok)
                   ? static_cast<double>(P.demand_in[slice * P.din_sn + key]) : 0.0;
  // the checkpoints are written only for a caller that keeps them (the
  // backward's input); an inference forward or prefill chunk passes none
  const bool ckpt = P.carry != nullptr;          // wave-uniform
  float* ccol = ckpt ? P.carry + slice * P.nb * T + min(key, T - 1) : nullptr;

  // staging: threads 0-255 one 16-byte chunk of the Q row tile; threads 0-31
  // the lse of its rows (+inf past the end: p = 0)
  const bool stager = threadIdx.x < 256;        // wave-uniform
  const int c256 = threadIdx.x & 255;
  bf16x8 rr = {};
  float lz = 0.f;
  const float* rmax = P.rmax + slice * P.C;
  const float* rden = P.rden + slice * P.C;
  auto fetch = [&](int rt) {
    const int64_t row0 = static_cast<int64_t>(rt) * kTileQ;
    const int64_t rows = min(max(C - row0, int64_t{0}), int64_t{kTileQ});
    if (stager)
      rr = buffer_load16<bf16x8>(make_rsrc(qs + row0 * D, rows * D * static_cast<int64_t>(sizeof(CT))),
                                 static_cast<uint32_t>(c256 * 16), 0);
    if (threadIdx.x < kTileQ) {
      const int64_t r = row0 + threadIdx.x;
      lz = r < C ? rmax[r] + __log2f(rden[r]) : INFINITY;
    }
  };
  auto stash = [&](int buf) {
    if (stager) {
      const int row = c256 / (D / 8), c = (c256 % (D / 8)) * 8;
      *reinterpret_cast<bf16x8*>(q_s[buf] + qs_slot(row) * TL::kKStride + c) = rr;
    }
    if (threadIdx.x < kTileQ) st_s[buf][threadIdx.x] = lz;
  };
  constexpr int kSteps = kTileQ / Mma<CT>::kStep;

  // the share tile of this wave's keys, staged for the product from the packed
  // transposed tile: fragment s of half h holds keys acc_row(8 s + t, h), two
  // runs of 4 consecutive keys (16 s + 4 h, 16 s + 8 + 4 h)
  auto stage_sh = [&](int buf, const bf16x8 (&xf)[2]) {
    CT* dst = sh_s[buf] + l32 * KG::kStride + wave * kTileK + 4 * h;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bf16x4 lo = {xf[s][0], xf[s][1], xf[s][2], xf[s][3]};
      const bf16x4 hi = {xf[s][4], xf[s][5], xf[s][6], xf[s][7]};
      *reinterpret_cast<bf16x4*>(dst + 16 * s) = lo;
      *reinterpret_cast<bf16x4*>(dst + 16 * s + 8) = hi;
    }
  };
  auto step = [&](int buf, int rt, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    RowFrag<CT, D> qf;
    lds_row_frag<CT, D>(qf, q_s[buf], l32, h);      // slot l32 holds row qsig(l32)
    const floatx16 sacc = mma_rows<CT, D>(qf, kf, floatx16{});
    float lzr[16];
    lds_read16(st_s[buf] + 16 * h, lzr);
    float p[16], x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[i], P.c, -lzr[i]));
    if constexpr (DIAG) {
      const int dk = l32 - 16 * h;                 // key - row(i) = dk - i on the diagonal tile
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dk > i) p[i] = 0.f;
    }
    const float cin = static_cast<float>(run);
    if (ckpt && h == 0 && key_ok) ccol[static_cast<int64_t>(rt) * T] = cin;   // the demand entering the tile
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = p[i];
    run += static_cast<double>(scan_incl_qs(x, cin + kEps, hf));      // demand + p + eps
#pragma unroll
    for (int i = 0; i < 16; ++i) p[i] *= fast_rcp(x[i]);               // share
    floatx16 xt = floatx16{};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) xt = Mma<CT>::mma(acc_frag<CT>(p, s), id_park[s][lane], xt);
    float xv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = xt[i];
    const bf16x8 xf[2] = {acc_frag<CT>(xv, 0), acc_frag<CT>(xv, 1)};
    stage_sh(buf, xf);
    // row sums of the staged (bf16) shares: each lane half adds its 16 keys of
    // the transposed tile on the VALU, then the halves (with the loop
    // unrolled: fwd_keyout -1.5% against all-ones MFMAs).  The transposed
    // registers already hold the bf16-rounded values exactly (the identity
    // product of bf16 operands is exact in fp32), so they are added as they
    // are: the same sums as of the staged values, without converting back.
    const HalfPair rp = halves(sum16(xv));
    if (h == 0) rs_s[buf][wave][l32] = rp.lo + rp.hi;
  };
  auto stage_zero = [&](int buf) {
    const bf16x8 z[2] = {bf16x8{}, bf16x8{}};
    stage_sh(buf, z);
    if (h == 0) rs_s[buf][wave][l32] = 0.f;
  };

  // share V of the group's KW * 32 keys for tile qt, formed by the last 8
  // waves: product wave pw forms rows 16 (pw & 1) + [0, 16) x head dims
  // 16 (pw >> 1) + [0, 16) over all the group's keys (with 16 waves, waves
  // 0-7 form none: each SIMD then holds two product waves and two others)
  const int pw = wave - (KW - 8);
  const bool prod_wave = pw >= 0;                // wave-uniform
  const int rh = pw & 1, dq4 = (pw >> 1) & 3;
  __bf16* op_s = op + slice * ntiles * (D * kTileQ);
  float* rp_s = rp + slice * ntiles * kTileQ;
  const int64_t gbase = cg.base(kg) - rt0;
  auto product = [&](int rt, int buf) {
    if (rt < 0) return;
    floatx4 acc = floatx4{};
    const CT* arow = sh_s[buf] + (16 * rh + (lane & 15)) * KG::kStride + 8 * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < KW; ++ks) {
      const bf16x8 av = *reinterpret_cast<const bf16x8*>(arow + kTileK * ks);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, vpark[dq4][ks][lane], acc, 0, 0, 0);
    }
    // output: lane <-> head dim 16 dq4 + (lane & 15), register j <-> row 16 rh + 4 (lane >> 4) + j;
    // the partial tile is stored in 16 x 16 blocks (part_block_off), streamed past the caches
    const int64_t tile = gbase + rt;
    const floatx2 a = {acc[0], acc[1]}, b = {acc[2], acc[3]};
    const bf16x2 pa = __builtin_convertvector(a, bf16x2), pb = __builtin_convertvector(b, bf16x2);
    const bf16x4 v = {pa[0], pa[1], pb[0], pb[1]};
    __builtin_nontemporal_store(__builtin_bit_cast(floatx2, v),
                                reinterpret_cast<floatx2*>(op_s + tile * (D * kTileQ) + part_block_off(dq4, rh, lane)));
    if (pw == 0 && lane < kTileQ) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) s += rs_s[buf][w][lane];
      __builtin_nontemporal_store(s, rp_s + tile * kTileQ + lane);
    }
  };

  fetch(rt0);
  if (P.v != nullptr) {
#pragma unroll
    for (int c = 0; c < kVChunks; ++c) {
      const int i = threadIdx.x + c * KG::kThreads;
      const int kk = i / (D / 8), d0 = (i % (D / 8)) * 8;           // key in the group, first head dim
      const int w = kk / kTileK, j = (kk % kTileK) / 8, t = kk % 8;
      // one 2-byte store per value (lanes write distinct halves of shared words)
      __bf16* dst = reinterpret_cast<__bf16*>(&vpark[d0 / 16][w][16 * j + d0 % 16]) + t;
#pragma unroll
      for (int e = 0; e < 8; ++e) dst[8 * e] = vfr[c][e];
    }
  } else {
#pragma unroll
    for (int u = 0; u < D / 16; ++u) vpark[u][wave][lane] = vfr[u];
  }
  if (wave == 0) {
#pragma unroll
    for (int s = 0; s < 2; ++s) id_park[s][lane] = ident_qs<CT>(l32, h, s);
  }
  stash(0);
  __syncthreads();
  // the product of tile qt - 1 (staged before the previous barrier, in the
  // other buffer) runs anywhere before this step's barrier, which the stage
  // of tile qt + 1 into that buffer follows.  Waves w and w + 4 share a SIMD:
  // product waves 4-7 form it before their step, 0-3 after their stash, so
  // the product waves of a SIMD leave each barrier out of phase (-7% on this
  // kernel at 8 waves)
  const bool early = prod_wave && pw >= 4, late = prod_wave && pw < 4;   // wave-uniform
  auto iter = [&](int j, int buf) __attribute__((always_inline)) {
    const int rt = rt0 + j;                      // chunk row tiles in causal order
    const int grt = q0t + rt;                    // its global row tile (diagonal: grt == kb)
    fetch(min(rt + 1, nq - 1));                  // the last step reloads its own tile, unused
    if (early) product(j > 0 ? rt - 1 : -1, buf ^ 1);
    if (active && grt >= kb) {
      if (grt > kb) step(buf, rt, std::false_type{});
      else step(buf, rt, std::true_type{});
    } else {
      stage_zero(buf);
    }
    stash(buf ^ 1);
    if (late) product(j > 0 ? rt - 1 : -1, buf ^ 1);
    sync_lds();
  };
  double_buffered<true>(0, nq - rt0, iter);      // unrolled by two: buffer offsets fold into the LDS instructions
  if (prod_wave) product(nq - 1, (nq - rt0 - 1) & 1);   // the last tile, staged before the final barrier
  if (h == 0 && key_ok) P.total[slice * P.tot_sn + key] = static_cast<float>(run);
}

// out = (sum over key groups of the share V partials) / (S + eps), S = the sum
// of the row-sum partials, both in key-group order; S is also the forward's
// ssum.  Grid: (query tiles, slices from slice0), the tiles with the most key
// groups first.  Thread t sums elements [8 t, 8 t + 8) of the partial tiles
// (one head dim, 8 rows: part_dim / part_row).
template <int D, int KW>
__global__ __launch_bounds__(kThreads) void fwd_out_reduce(const __bf16* __restrict__ op,
                                                           const float* __restrict__ rp, int64_t ntiles,
                                                           int64_t T, int64_t Tk, float* __restrict__ out,
                                                           int64_t o_sn, float* __restrict__ ssum, int64_t slice0) {
  // T: the chunk's rows; Tk: keys (the chunk starts at row Tk - T)
  static_assert(D * kTileQ == 8 * kThreads, "one 16-byte chunk of the partial tile per thread");
  __shared__ float sum_s[D][kTileQ + 1];
  __shared__ float s_s[kTileQ];
  const int64_t slice = slice0 + blockIdx.y;
  using KG = KeyGroups<KW>;
  const ChunkGroups<KW> cg{(T + kTileQ - 1) / kTileQ, (Tk - T) / KG::kKeys};
  const int nq = static_cast<int>(cg.nq);
  const int tq = nq - 1 - static_cast<int>(blockIdx.x);
  const int ng = static_cast<int>(min(KG::groups(Tk) - 1, cg.a + tq / KW)) + 1;
  const int t = threadIdx.x;
  const __bf16* base = op + slice * ntiles * (D * kTileQ) + 8 * t;
  auto tile_of = [&](int g) { return cg.base(g) + tq - cg.first(g); };
  // groups in order, eight partial tiles in flight; threads 0-31 load the
  // same groups' row sums beside them (both added in group order)
  const bool srow = t < kTileQ;
  const float* gp = rp + slice * ntiles * kTileQ + (srow ? t : 0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float s = 0.f;
  for (int g = 0; g < ng; g += 8) {
    bf16x8 v[8];
    float r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (g + u < ng) {
        v[u] = load_once(base + tile_of(g + u) * (D * kTileQ));
        if (srow) r[u] = load_once(gp + tile_of(g + u) * kTileQ);
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (g + u < ng) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += static_cast<float>(v[u][e]);
        if (srow) s += r[u];
      }
    }
  }
  {
    // the thread's 8 elements: one head dim, 8 consecutive rows of the tile
    const int pd = part_dim(8 * t), pr = part_row(8 * t);
#pragma unroll
    for (int e = 0; e < 8; ++e) sum_s[pd][pr + e] = acc[e];
  }
  if (srow) {
    s_s[t] = s;
    const int64_t row = static_cast<int64_t>(tq) * kTileQ + t;
    if (row < T) ssum[slice * T + row] = s;
  }
  __syncthreads();
  // output rows: thread t takes row t / 8, head dims 8 (t % 8) + [0, 8)
  const int row = t / (D / 8), d8 = (t % (D / 8)) * 8;
  const int64_t grow = static_cast<int64_t>(tq) * kTileQ + row;
  if (grow < T) {
    const float inv = 1.f / (s_s[row] + kEps);
    floatx4 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = sum_s[d8 + e][row] * inv;
      b[e] = sum_s[d8 + 4 + e][row] * inv;
    }
    floatx4* o = reinterpret_cast<floatx4*>(out + slice * o_sn + grow * D + d8);
    o[0] = a;
    o[1] = b;
  }
}

// ---------------------------------------------------------------------------
// host side

// The key-parallel output pass replaces fwd_demand + fwd_out where it serves:
// bf16 operands, head_dim 64, the production operator, a chunk that starts at
// a multiple of 512 keys (the training forward, chunked prefill at such
// starts), one slice's partials (~0.5 byte per causal score element) within
// the budget.  The workspace holds the partials of as many slices as the
// budget allows, and the pass and its reduction run over the slices in
// batches of that many (a single batch at every training and prefill shape of
// the benchmark: one slice's partials are 35 MB at T = 16384).  512-key groups
// (16 waves); DILUTION_FORWARD_KEY_PASS=0 turns it off (read once by each call
// and by each size query: ForwardArgs::key_pass).
constexpr int64_t kKeyoutBudgetBytes = int64_t{24} << 30;
constexpr int kKeyoutWaves = 16;

inline int64_t keyout_tiles(int64_t C, int64_t Tk) {
  using KG = KeyGroups<kKeyoutWaves>;
  const ChunkGroups<kKeyoutWaves> cg{(C + kTileQ - 1) / kTileQ, (Tk - C) / KG::kKeys};
  return cg.base(KG::groups(Tk));
}
inline int64_t keyout_partial_bytes(int64_t n, int64_t C, int64_t Tk, int D) {
  return n * keyout_tiles(C, Tk) * (static_cast<int64_t>(D) * kTileQ * 2 + kTileQ * 4);
}
inline bool keyout_eligible(int64_t C, int64_t Tk, int64_t q0, int D, int prec, bool requested) {
  return requested && prec == 2 && D == 64 && q0 + C == Tk && q0 % KeyGroups<kKeyoutWaves>::kKeys == 0 &&
         keyout_partial_bytes(1, C, Tk, D) <= kKeyoutBudgetBytes;
}
// slices per key-pass batch: all of them when their partials fit the budget,
// else as many batches as the budget needs, of equal size (a last batch of a
// slice or two would leave most CUs idle behind its longest walks)
inline int64_t keyout_batch(int64_t n, int64_t C, int64_t Tk, int D) {
  const int64_t per = keyout_partial_bytes(1, C, Tk, D);
  int64_t fit = per > 0 ? kKeyoutBudgetBytes / per : n;
  fit = fit < 1 ? 1 : (fit < n ? fit : n);
  const int64_t batches = (n + fit - 1) / fit;
  return (n + batches - 1) / batches;
}

struct FwdWorkspace {
  size_t vt, kt, qc, kc, op, rp, total;
};

FwdWorkspace fwd_layout(int64_t n, int64_t C, int64_t Tk, int D, int dtype, int prec, int want_pk,
                        bool key_pass) {
  const size_t ct = prec == 2 ? 2 : 4;
  const bool convert = dtype != native_dtype(prec);
  FwdWorkspace w{};
  const size_t tsz = align_up(ct * n * D * pad64(Tk));
  w.vt = 0;
  w.kt = w.vt + tsz;
  w.qc = w.kt + (want_pk ? tsz : 0);
  w.kc = w.qc + (convert ? align_up(ct * n * C * D) : 0);
  w.op = w.kc + (convert ? align_up(ct * n * Tk * D) : 0);
  w.rp = w.op;
  w.total = w.op;
  // the key pass's partials, when a chunk of this shape can take it (every
  // call is a chunk of rows [Tk - C, Tk) against keys [0, Tk))
  if (keyout_eligible(C, Tk, Tk - C, D, prec, key_pass)) {
    const int64_t nb = keyout_batch(n, C, Tk, D);
    w.rp = w.op + align_up(static_cast<size_t>(nb * keyout_tiles(C, Tk) * D * kTileQ * 2));
    w.total = w.rp + align_up(static_cast<size_t>(nb * keyout_tiles(C, Tk) * kTileQ * 4));
  }
  return w;
}

template <typename CT, int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
int launch_forward(const ForwardArgs& a) {
  const FwdWorkspace w = fwd_layout(a.n, a.C, a.Tk, D, a.dtype, kOperandPrec<CT>, a.pk != nullptr, a.key_pass);
  char* ws = static_cast<char*>(a.workspace);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const bool convert = a.dtype != kNativeDtype<CT>;
  const int64_t tk_pad = pad64(a.Tk);

  CT* vt = reinterpret_cast<CT*>(ws + w.vt);
  CT* kt = a.pk ? reinterpret_cast<CT*>(ws + w.kt) : nullptr;
  CT* qc = convert ? reinterpret_cast<CT*>(ws + w.qc) : nullptr;
  CT* kc = convert ? reinterpret_cast<CT*>(ws + w.kc) : nullptr;
  // the key pass parks V from the caller's bf16 rows: no V^T to write (the
  // workspace keeps its room, shared with the three-pass forward's layout)
  constexpr bool kKeyPassBuilt =
      std::is_same_v<CT, __bf16> && D == 64 && BID == BID_SOFTMAX && SHARE == SHARE_INCL;
  const bool key_pass = kKeyPassBuilt && keyout_eligible(a.C, a.Tk, a.q0, D, kOperandPrec<CT>, a.key_pass);
  const bool v_rows = key_pass && !convert;

  // operands in the compute type; V^T (and K^T) tiles
  const unsigned ktiles = static_cast<unsigned>(tk_pad / 64);
  const unsigned qtiles = static_cast<unsigned>(pad64(a.C) / 64);
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    PrepJobs kv{};
    unsigned nkv = 0;
    if (!v_rows) kv.job[nkv++] = PrepJob{a.v, a.kv_sn, nullptr, 0, vt, nullptr};
    if (convert || kt != nullptr) kv.job[nkv++] = PrepJob{a.k, a.kv_sn, kc, a.Tk * D, kt, nullptr};
    if (nkv > 0)
      DIL_TIMED("prep", st, (prep_kernel<CT, D><<<dim3(ktiles, ns, nkv), kThreads, 0, st>>>(
                                kv, a.dtype, a.Tk, D * tk_pad, tk_pad, s0)));
    if (convert) {
      PrepJobs qj{};
      qj.job[0] = PrepJob{a.q, a.q_sn, qc, a.C * D, nullptr, nullptr};
      DIL_TIMED("prep", st, (prep_kernel<CT, D><<<dim3(qtiles, ns, 1), kThreads, 0, st>>>(qj, a.dtype, a.C, 0, 0, s0)));
    }
  });

  FwdParams P{};
  P.q = convert ? static_cast<const void*>(qc) : a.q;
  P.q_sn = convert ? a.C * D : a.q_sn;
  P.k = convert ? static_cast<const void*>(kc) : a.k;
  P.k_sn = convert ? a.Tk * D : a.kv_sn;
  P.v = v_rows ? a.v : nullptr;
  P.v_sn = a.kv_sn;
  P.vt = vt;
  P.kt = kt;
  P.t_sn = D * tk_pad;
  P.tk_pad = tk_pad;
  P.C = a.C;
  P.Tk = a.Tk;
  P.q0 = a.q0;
  P.nb = (a.C + kTileQ - 1) / kTileQ;
  // longest first pays where the items' weights differ widely: a chunk that
  // starts before its own length (training, a first prefill chunk)
  P.lpt = a.q0 < a.C && longest_first_for(a.n, a.Tk);
  P.scale = 1.f / sqrtf(static_cast<float>(D));
  P.c = kLog2e * P.scale;
  P.out = a.out;
  P.o_sn = a.o_sn;
  P.rmax = a.rmax;
  P.rden = a.rden;
  P.ssum = a.ssum;
  P.carry = a.carry;
  P.demand_in = a.demand_in;
  P.din_sn = a.din_sn;
  P.total = a.total;
  P.tot_sn = a.tot_sn;
  P.pk = a.pk;
  P.shift = a.var.shift;
  P.lshift = log2f(a.var.shift);

  P.n = a.n;
  P.groups = static_cast<int>((a.C + 4 * kTileQ - 1) / (4 * kTileQ));
  const dim3 grid(static_cast<unsigned>(xcd_grid(P.groups * a.n)));
  if (a.pk) DIL_TIMED("fwd_stats", st, (fwd_stats<CT, D, true, BID><<<grid, kThreads, 0, st>>>(P)));
  else DIL_TIMED("fwd_stats", st, (fwd_stats<CT, D, false, BID><<<grid, kThreads, 0, st>>>(P)));
  if constexpr (kKeyPassBuilt) {
    if (key_pass) {
      // one key pass forms the checkpoints, the totals and the share V
      // partials; the reduction finishes out and ssum
      __bf16* op = reinterpret_cast<__bf16*>(ws + w.op);
      float* rp = reinterpret_cast<float*>(ws + w.rp);
      constexpr int KW = kKeyoutWaves;
      using KG = KeyGroups<KW>;
      const unsigned nq = static_cast<unsigned>((a.C + kTileQ - 1) / kTileQ);
      const int64_t ntiles = keyout_tiles(a.C, a.Tk);
      P.kgroups = static_cast<int>(KG::groups(a.Tk));
      // longest walks first, group by group, whatever the size: every chunk's
      // walks differ in length (its diagonal groups are shorter), and in slice
      // order a CU could finish a whole walk after the rest (a prefill chunk of
      // 256 slices at 2048 rows ended ~0.17 ms after its work would balance)
      P.lpt = 1;
      // slices in batches whose partials fit the workspace (one batch at
      // every benchmark shape); each batch's pass and reduction see only its
      // slices, through pointers advanced to its first slice
      const int64_t batch = keyout_batch(a.n, a.C, a.Tk, D);
      for (int64_t b0 = 0; b0 < a.n; b0 += batch) {
        const int64_t nbat = min(batch, a.n - b0);
        FwdParams B = P;
        B.n = nbat;
        B.q = static_cast<const CT*>(P.q) + b0 * P.q_sn;
        B.k = static_cast<const CT*>(P.k) + b0 * P.k_sn;
        if (P.v != nullptr) B.v = static_cast<const CT*>(P.v) + b0 * P.v_sn;
        B.vt = static_cast<const CT*>(P.vt) + b0 * P.t_sn;
        B.rmax = P.rmax + b0 * P.C;
        B.rden = P.rden + b0 * P.C;
        if (P.carry != nullptr) B.carry = P.carry + b0 * P.nb * P.Tk;
        if (P.demand_in != nullptr) B.demand_in = P.demand_in + b0 * P.din_sn;
        B.total = P.total + b0 * P.tot_sn;
        const dim3 gko(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(B.kgroups) * nbat)));
        DIL_TIMED("fwd_keyout", st, (fwd_keyout<D, KW><<<gko, KG::kThreads, 0, st>>>(B, op, rp, ntiles)));
        float* out_b = a.out + b0 * a.o_sn;
        float* ssum_b = a.ssum + b0 * a.C;
        slice_batches(nbat, [&](int64_t s0, unsigned ns) {
          DIL_TIMED("fwd_out_reduce", st,
                    (fwd_out_reduce<D, KW><<<dim3(nq, ns), kThreads, 0, st>>>(op, rp, ntiles, a.C, a.Tk, out_b,
                                                                             a.o_sn, ssum_b, s0)));
        });
      }
      return static_cast<int>(hipGetLastError());
    }
  }
  P.kgroups = static_cast<int>((a.Tk + 4 * kTileK - 1) / (4 * kTileK));
  DIL_TIMED("fwd_demand", st,
            (fwd_demand<CT, D, BID><<<dim3(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(P.kgroups) * a.n))),
                                      kThreads, 0, st>>>(P)));
  DIL_TIMED("fwd_out", st, (fwd_out<CT, D, BID, SHARE><<<grid, kThreads, 0, st>>>(P)));
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace dil
