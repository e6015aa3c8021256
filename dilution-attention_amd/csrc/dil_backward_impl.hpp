// Backward of the dilution-attention operator.
//
// Reference behaviour: _DilutionAttentionFn.backward,
// /root/reference/src/dilution/kernels.py:851-903, and the decomposition in
// /root/reference/docs/kernels.md:62-84.  With s = 1/sqrt(d), C the inclusive
// column demand (c + p) and S the row sum of shares:
//
//   ds_ij  = (dO_i . v_j - dO_i . o_i) / (S_i + eps) = dO'_i . v_j - dbs_i,
//            dO'_i = dO_i sinv_i (the rows of dO prescaled once), sinv_i = 1/(S_i+eps)
//   inv_ij = 1 / (C_ij + eps),   sh_ij = p_ij inv_ij
//   g_ij   = ds_ij sh_ij inv_ij                  (adjoint flowing into the demand)
//   G_ij   = sum_{i' >= i} g_i'j                 (inclusive reverse column scan)
//   dp_ij  = ds_ij inv_ij - G_ij,   p dp = ds_ij sh_ij - p_ij G_ij
//   ghat_i = sum_j (p dp)_ij,   da_ij = (p dp)_ij - p_ij ghat_i
//   dq = s da K,   dk = s da^T Q,   dv = sh^T dO' 
//
// Kernels (gfx950, deterministic, no atomics; tiles in the query-split layout
// of dil_tiles.hpp, causal diagonal tiles peeled out of the main loops):
//   bwd_rows    per row: lse = rmax + log2 rden, sinv = 1/(S + eps),
//               dbs = (dO . o) sinv; and dO' = dO sinv in the compute type,
//               row-major and transposed, from the same read of dO.
//   bwd_key     one wave per 32-key tile, query tiles walked in reverse:
//               dv += sh^T dO' and dk_main += (p dp)^T Q on MFMA with
//               keys in lanes; the running suffix G per key is stored at every
//               tile boundary for bwd_query.
//   bwd_query   one wave per 32-row tile over its causal key tiles: the same
//               chain with G from the checkpoints; (p dp) transposed by an
//               identity MFMA so dq += (p dp) K runs with queries in lanes,
//               and ghat (the row sums of p dp) summed from the transposed
//               registers; dq = s dq_main - ghat pk.  bf16 up to head_dim 64
//               keeps dO' and the identity in LDS: three workgroups per CU.
//   prep_ghat_q (ghat * Q)^T tiles for the correction.
//   bwd_dkcorr  one wave per key tile: dk = s dk_main - s sum_i p_ij (ghat_i q_i).
//   bwd_keyq    (bf16 operands, head_dim 64) bwd_key and bwd_query's dq in one
//               walk of 256 keys per workgroup: dq partials per key group,
//               summed in order by bwd_dq_reduce, which also writes the
//               (ghat * Q)^T tiles; it replaces bwd_key, bwd_query and
//               prep_ghat_q for every bid / share pair.
#pragma once

#include "dil_common.hpp"
#include "dil_internal.hpp"
#include "dil_tiles.hpp"
#include "dil_variant.hpp"

#include <algorithm>
#include <type_traits>

namespace dil {

namespace {

struct BwdParams {
  const void* q;      // CT rows (n, T, D)
  const void* k;
  const void* v;
  const void* dout;   // CT rows
  const void* qt;     // CT transposed copies, tile-major (T_pad rows per slice)
  const void* kt;
  const void* dot;
  const void* qgt;    // CT (ghat * q)^T, tile-major
  int64_t T, t_pad, nb;
  int64_t n;          // slices
  int kgroups;        // groups of 4 tiles (128 keys or rows) per slice
  float c, scale;
  const float* lse;   // (n, T): log2-sum-exp of the row, or r0 of the variant's bid
  const float* rb1;   // (n, T): r1 of the variant's bid (ratio bids), else null
  float lshift;       // log2(SHIFT)
  const float* sinv;
  const float* dbs;
  float* ghat;        // (n, T)
  const float* carry; // (n, nb, T)
  float* sufk;        // (n, nb, T)
  float* dkm;         // (n, T, D) fp32: sum_i (p dp)_ij q_i
  const float* pk;    // (n, T, D)
  void* dq;
  void* dk;
  void* dv;
  int gdt;            // grad dtype
  int lpt;            // dispatch longest first (xcd_work_item)
};

// ---------------------------------------------------------------------------
// per-row prologue

template <typename CT, int D, int BID = BID_SOFTMAX>
__global__ __launch_bounds__(kThreads) void bwd_rows(const void* __restrict__ dout, int ddt,
                                                     const float* __restrict__ out,
                                                     const float* __restrict__ rmax,
                                                     const float* __restrict__ rden,
                                                     const float* __restrict__ ssum, float* __restrict__ lse,
                                                     float* __restrict__ sinv, float* __restrict__ dbs,
                                                     float* __restrict__ rb1, int64_t T, int64_t t_pad,
                                                     CT* __restrict__ doc, CT* __restrict__ dot,
                                                     int64_t slice0) {
  // Grid: (64-row tiles, slices from slice0).  A row's D / 8 lanes are
  // consecutive; each holds 8 elements of dO and o.
  constexpr int kVecPerRow = D / 8;
  __shared__ float tile[64][D + 1];
  const int64_t slice = slice0 + blockIdx.y;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
  // 64 * D / 8 items are a whole number of waves: each shuffle below runs on
  // full waves
  for (int idx = threadIdx.x; idx < 64 * kVecPerRow; idx += kThreads) {
    const int r = idx / kVecPerRow, sub = idx % kVecPerRow, c8 = sub * 8;
    const bool ok = r0 + r < T;
    const int64_t row = slice * T + r0 + r;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float acc = 0.f;
    if (ok) {
      float o[8];
      load8_f32(dout, row * D + c8, ddt, v);
      load8_f32(out, row * D + c8, DT_F32, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc = fmaf(v[e], o[e], acc);
    }
#pragma unroll
    for (int m = 1; m < kVecPerRow; m <<= 1) acc += __shfl_xor(acc, m, 64);
    if (ok) {
      const float si = 1.f / (ssum[row] + kEps);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= si;
      if (sub == 0) {
        if constexpr (BID == BID_SOFTMAX) {
          lse[row] = rmax[row] + __log2f(rden[row]);
        } else {
          float a0, a1;
          bid_row_params<BID>(rmax[row], rden[row], static_cast<float>(r0 + r + 1), true, a0, a1);
          lse[row] = a0;
          rb1[row] = a1;
        }
        sinv[row] = si;
        dbs[row] = acc * si;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][c8 + e] = v[e];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 64 * kVecPerRow; idx += kThreads) {
    const int r = idx / kVecPerRow, c8 = (idx % kVecPerRow) * 8;
    if (r0 + r < T) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[r][c8 + e];
      store8<CT>(doc + (slice * T + r0 + r) * D + c8, v);
    }
  }
  // transposed: item idx is 32-row half b, column c, rows r8 .. r8 + 7 of it
  for (int idx = threadIdx.x; idx < 8 * D; idx += kThreads) {
    const int b = idx / (4 * D), c = (idx % (4 * D)) >> 2, r8 = 32 * b + (idx & 3) * 8;
    if (r0 + r8 < t_pad) {
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[r8 + e][c];
      store8<CT>(dot + slice * D * t_pad + tmajor_index(r0 + r8, c, D), v);
    }
  }
}

// (ghat * q)^T in the compute type from the tile-major transposed copy Q^T
// (n, t_pad rows), whose padding rows are zero.  One workgroup per 32-row
// tile; each thread scales 8 consecutive elements (8 rows of one column) with
// one 16-byte load and store.
template <typename CT, int D>
__global__ __launch_bounds__(kThreads) void prep_ghat_q(const CT* __restrict__ qt,
                                                        const float* __restrict__ ghat, int64_t T,
                                                        int64_t t_pad, CT* __restrict__ dst, int64_t slice0) {
  __shared__ float g_s[32];
  const int64_t slice = slice0 + blockIdx.y;
  const int64_t row0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t base = slice * D * t_pad + row0 * D;
  if (threadIdx.x < 32) {
    const int64_t row = row0 + threadIdx.x;
    g_s[threadIdx.x] = row < T ? ghat[slice * T + row] : 0.f;
  }
  __syncthreads();
  for (int e8 = threadIdx.x * 8; e8 < 32 * D; e8 += kThreads * 8) {
    float v[8];
    load8<CT>(qt + base + e8, v);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] *= g_s[(e8 & 31) + k];
    store8<CT>(dst + base + e8, v);
  }
}

// Per-row statistics of one 32-row tile staged in LDS: up to three arrays of
// 32 floats, the second one negated (-dO.o/(S+eps) is the initial value of
// the dO V^T products).  Rows past the end read +inf from the first array,
// so that p = 0, and 0 from the others.
// With CLAMP every thread loads (from a clamped row) and the value is fixed up
// in store(); without it only the threads that store load.
template <int NARR, bool CLAMP = true>
struct RowStatsLoader {
  float r;
  bool ok;
  float pad0 = INFINITY;                     // first array past the end (p = 0 there)
  __device__ void load(const float* a, const float* b, const float* c, int64_t row0, int64_t T) {
    const int t = threadIdx.x;
    const float* src = t < kTileQ ? a : (t < 2 * kTileQ ? b : c);
    const int64_t row = row0 + (t % kTileQ);
    ok = row < T;
    if (CLAMP) r = src[min(row, T - 1)];
    else r = (ok && t < NARR * kTileQ) ? src[row] : 0.f;
  }
  __device__ void store(float* lds) const {
    const int t = threadIdx.x;
    if (t < NARR * kTileQ) {
      const float v = ok ? r : (t < kTileQ ? pad0 : 0.f);
      lds[t] = (t >= kTileQ && t < 2 * kTileQ) ? -v : v;
    }
  }
  // every thread writes (threads past the arrays into padding, lds holding
  // kThreads floats): no exec-masked branch around the wait for the load
  __device__ void store_all(float* lds) const {
    const int t = threadIdx.x;
    const float v = ok ? r : (t < kTileQ ? pad0 : 0.f);
    lds[t] = (t >= kTileQ && t < 2 * kTileQ) ? -v : v;
  }
};


template <typename CT, int D>
constexpr int bwd_occupancy() {
  return (sizeof(CT) == 2 && D <= 64) ? 2 : 1;
}

// bwd_query's parked form keeps its dO' operands and the transpose identity
// in LDS and sums ghat on the VALU, which leaves room for three workgroups per
// CU (<= 168 VGPRs, 48 KB of LDS each) with bf16 operands up to head_dim 64:
// -16% at T = 2048, -10% at 4096 and 16384 against the register form (ones
// column MFMA for ghat, two workgroups per CU), which runs for head_dim 128
// and the operator variants.  With fp32 or split operands (head_dim <= 64)
// the parked form is 8 waves (256 rows) per workgroup: <= 256 registers a
// lane (two waves per SIMD, where the register form holds one) and ~124 KB
// of LDS (the parked dO' of 8 waves and one set of K / V / K^T stages for
// all of them), one workgroup per CU.
template <typename CT, int D>
constexpr bool query_parks() {
  return D <= 64;
}
template <typename CT, int D>
constexpr int query_waves() {
  return sizeof(CT) == 2 ? 4 : 8;
}

// ---------------------------------------------------------------------------
// key-parallel reverse pass: dv, dk_main, suffix checkpoints

// At head_dim 256 the dk and dv accumulators of a wave's 32 keys (256 fp32
// registers a lane) do not fit beside the key and value fragments and the
// chain: SPLIT workgroups then share a key group, each accumulating dk and dv
// for D / SPLIT of the head dims while recomputing the whole chain (the score
// products run over all D).  The first of them stores the suffix checkpoints.
template <typename CT, int D> constexpr int key_split() { return D > 128 ? 2 : 1; }

template <typename CT, int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
__global__ __launch_bounds__(kThreads, (bwd_occupancy<CT, D>())) void bwd_key(BwdParams P) {
  using TL = Tiles<CT, D>;
  constexpr int kSplit = key_split<CT, D>();
  constexpr int kDH = D / kSplit;                     // head dims of dk / dv this workgroup forms
  constexpr int kDT = kDTiles<kDH>;                   // ... in 32-dim tiles
  constexpr int kNS = BID == BID_SOFTMAX ? 2 : 3;                // per-row statistics staged
  __shared__ __attribute__((aligned(16))) CT q_s[2][kTileQ * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT do_s[2][kTileQ * TL::kKStride];
  // the transposed row tiles hold the workgroup's kDH head dims only
  __shared__ __attribute__((aligned(16))) CT qt_s[2][kDH * TL::kTStride];
  __shared__ __attribute__((aligned(16))) CT dot_s[2][kDH * TL::kTStride];
  // lse (r0), -dbs, r1, then padding: every thread of the stash writes a slot
  __shared__ __attribute__((aligned(16))) float st_s[2][kThreads];
  __shared__ float cs_s[2][kThreads];             // demand checkpoints of the 128 keys, then padding

  // early keys (long walks) first; with a head-dim split, both parts of a
  // key group go out together
  const WorkItem item = xcd_work_item(P.kgroups * kSplit, P.n, false, P.lpt != 0);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const float hf = static_cast<float>(h);
  const int part = item.idx % kSplit;            // which D / kSplit head dims of dk and dv
  const int t0 = part * kDT;                     // first 32-dim tile of them
  const int kb0 = (item.idx / kSplit) * 4;
  const int kb = kb0 + wave;                     // key tile of this wave
  const int64_t key = static_cast<int64_t>(kb) * kTileK + l32;
  const int nq = static_cast<int>((P.T + kTileQ - 1) / kTileQ);
  const bool active = static_cast<int64_t>(kb) * kTileK < P.T;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.T * D;
  const CT* dos = static_cast<const CT*>(P.dout) + slice * P.T * D;
  const CT* qts = static_cast<const CT*>(P.qt) + slice * D * P.t_pad;
  const CT* dots = static_cast<const CT*>(P.dot) + slice * D * P.t_pad;
  const float* lse = P.lse + slice * P.T;
  const float* dbs = P.dbs + slice * P.T;

  // this wave's keys as B operands (lane <-> key)
  RowFrag<CT, D> kf, vf;
  if (key < P.T) {
    load_row_frag<CT, D>(kf, static_cast<const CT*>(P.k) + (slice * P.T + key) * D + h * (D / 2));
    load_row_frag<CT, D>(vf, static_cast<const CT*>(P.v) + (slice * P.T + key) * D + h * (D / 2));
  } else {
    zero_row_frag<CT, D>(kf);
    zero_row_frag<CT, D>(vf);
  }
  floatx16 dka[kDT], dva[kDT];
#pragma unroll
  for (int t = 0; t < kDT; ++t) {
    dka[t] = floatx16{};
    dva[t] = floatx16{};
  }
  float sufk = 0.f;
  float* sufk_col = P.sufk + slice * P.nb * P.T + key;
  const bool store_suffix = part == 0;           // wave-uniform

  // a stage: the Q and dO' row tiles, their transposes, the row statistics and
  // the demand checkpoints of the workgroup's 128 keys entering the tile
  KTileLoader<CT, D, true> ql, dl;        // row tiles in query-split slot order
  TTileLoader<CT, kDH, kLoadBuffer, D> qtl, dtl;   // head dims [t0 * 32, t0 * 32 + kDH) of the transposes
  RowStatsLoader<kNS> sl;
  if constexpr (!bid_log2<BID>()) sl.pad0 = 0.f;
  const int64_t ck = static_cast<int64_t>(kb0) * kTileK + (threadIdx.x & (4 * kTileK - 1));
  const bool ck_ok = ck < P.T;
  const float* ccol = P.carry + slice * P.nb * P.T + min(ck, P.T - 1);
  float cr = 0.f;
  const int64_t t_off = static_cast<int64_t>(t0) * 32 * kTileK;   // the first taken head dim within a tile
  auto fetch = [&](int qt) {
    const int64_t row0 = static_cast<int64_t>(qt) * kTileQ;
    ql.load(qs, row0, P.T);
    dl.load(dos, row0, P.T);
    qtl.load(qts + t_off, row0);
    dtl.load(dots + t_off, row0);
    sl.load(lse, dbs, BID == BID_SOFTMAX ? dbs : P.rb1 + slice * P.T, row0, P.T);
    cr = ccol[static_cast<int64_t>(qt) * P.T];
  };
  auto stash = [&](int buf) {
    ql.store(q_s[buf]);
    dl.store(do_s[buf]);
    qtl.store(qt_s[buf]);
    dtl.store(dot_s[buf]);
    sl.store_all(st_s[buf]);
    cs_s[buf][threadIdx.x] = ck_ok ? cr : 0.f;
  };
  constexpr int kSteps = kTileQ / Mma<CT>::kStep;

  auto step = [&](int qt, int buf, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const float* st = st_s[buf];
    const float cin = cs_s[buf][wave * kTileK + l32];   // demand entering the tile
    float lz[16], ndb[16];
    lds_read16(st + kTileQ + 16 * h, ndb);
    // both score-shaped products first; ds = dO' V^T - dbs starts from -dbs
    // and runs under the p / demand chain.  Slot l32 of a row tile holds row
    // qsig(l32); with a head-dim split (head_dim 256) the Q and dO' operands
    // are read per instruction instead of whole
    floatx16 sacc, dov;
    if constexpr (kSplit > 1) {
      const int off = l32 * TL::kKStride + h * (D / 2);
      sacc = mma_rows_src<CT, D>(q_s[buf] + off, kf, floatx16{});
      dov = mma_rows_src<CT, D>(do_s[buf] + off, vf, as_x16(ndb));
    } else {
      RowFrag<CT, D> qf, dof;
      lds_row_frag<CT, D>(qf, q_s[buf], l32, h);
      lds_row_frag<CT, D>(dof, do_s[buf], l32, h);
      sacc = mma_rows<CT, D>(qf, kf, floatx16{});
      dov = mma_rows<CT, D>(dof, vf, as_x16(ndb));
    }
    lds_read16(st + 16 * h, lz);
    float p[16], x[16], jac[16];
    if constexpr (BID == BID_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[i], P.c, -lz[i]));
    } else {
      float r1[16];
      lds_read16(st + 2 * kTileQ + 16 * h, r1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = bid_p<BID>(sacc[i], P.c, P.scale, lz[i], r1[i], P.lshift);
        jac[i] = bid_jac<BID>(p[i], sacc[i], P.scale, lz[i]);
      }
    }
    if constexpr (DIAG) {
      const int dk = l32 - 16 * h;               // key - row(i) = dk - i on the diagonal tile
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dk > i) {
          p[i] = 0.f;
          jac[i] = 0.f;
        }
    }
    float sh[16], w[16];
    if constexpr (SHARE != SHARE_NONE) {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = p[i];
      if constexpr (SHARE == SHARE_EXCL) scan_excl_qs(x, cin + kEps, hf);   // demand + eps
      else scan_incl_qs(x, cin + kEps, hf);                                // demand + p + eps
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = fast_rcp(x[i]);                   // inv
        sh[i] = p[i] * x[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) sh[i] = p[i];
    }
    // dv^T += dO'^T sh  (keys in lanes; dO' carries the 1/(S+eps) of A)
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto bfr = acc_frag<CT>(sh, s);
#pragma unroll
      for (int t = 0; t < kDT; ++t)
        dva[t] = Mma<CT>::mma(lds_tq_frag<CT, kDH>(dot_s[buf], 32 * t + l32, h, s), bfr, dva[t]);
    }
    if constexpr (is_production<BID, SHARE>()) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        w[i] = dov[i] * sh[i];                   // ds sh
        x[i] = w[i] * x[i];                      // g = ds sh inv
      }
      sufk += scan_suffix_qs(x, sufk, hf);       // x = G
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] = fmaf(-p[i], x[i], w[i]);   // p dp = ds sh - p G
    } else {
      // dp = ds inv - G (+ g for the exclusive share; ds with no share step);
      // the MFMA operand is jac dp (jac = p for the softmax bids)
      if constexpr (SHARE != SHARE_NONE) {
        float g[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          w[i] = dov[i] * x[i];                  // ds inv
          g[i] = w[i] * sh[i];                   // ds sh inv
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = g[i];
        sufk += scan_suffix_qs(x, sufk, hf);     // x = G
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          w[i] -= x[i];
          if constexpr (SHARE == SHARE_EXCL) w[i] += g[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = dov[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] *= bid_log2<BID>() ? p[i] : jac[i];
    }
    // dk_main^T += Q^T (p dp)
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto bfr = acc_frag<CT>(w, s);
#pragma unroll
      for (int t = 0; t < kDT; ++t)
        dka[t] = Mma<CT>::mma(lds_tq_frag<CT, kDH>(qt_s[buf], 32 * t + l32, h, s), bfr, dka[t]);
    }
  };

  fetch(nq - 1);
  stash(0);
  __syncthreads();
  // vmcnt counts stores as well as loads, so the compiler must know on every
  // path how many memory operations follow the fetched data when the stash
  // waits for it: the stash is unconditional (the last iteration stashes into
  // the idle buffer), every thread writes LDS in it, and the step's suffix
  // checkpoint is stored after it (stored inside the conditional step, the
  // wait would also wait for that store).
  auto iter = [&](int j, int buf) __attribute__((always_inline)) {
    const int qt = nq - 1 - j;                   // query tiles in reverse
    fetch(max(qt - 1, kb0));                     // the last step reloads its own tile, unused
    const bool run = active && qt >= kb;
    const float sufk_in = sufk;                  // suffix entering this tile from below
    if (run) {
      if (qt > kb) step(qt, buf, std::false_type{});
      else step(qt, buf, std::true_type{});
    }
    stash(buf ^ 1);
    if (run && store_suffix && h == 0 && key < P.T) sufk_col[static_cast<int64_t>(qt) * P.T] = sufk_in;
    sync_lds();
  };
  double_buffered<true>(0, nq - kb0, iter);

  if (key < P.T) {
    // registers 4 j .. 4 j + 3 hold four consecutive head dims (acc_row)
    float* dkrow = P.dkm + (slice * P.T + key) * D;
    const int64_t dvrow = (slice * P.T + key) * D;
#pragma unroll
    for (int t = 0; t < kDT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * (t0 + t) + acc_row(4 * j, h);
        if (d < D) {
          *reinterpret_cast<floatx4*>(dkrow + d) =
              floatx4{dka[t][4 * j], dka[t][4 * j + 1], dka[t][4 * j + 2], dka[t][4 * j + 3]};
          store4_as(P.dv, dvrow + d, P.gdt,
                    floatx4{dva[t][4 * j], dva[t][4 * j + 1], dva[t][4 * j + 2], dva[t][4 * j + 3]});
        }
      }
  }
}

// ---------------------------------------------------------------------------
// row-parallel dq pass

template <typename CT, int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL, bool PARK = false,
          int W = 4>
__global__ __launch_bounds__(64 * W, ((PARK && query_parks<CT, D>()) ? (W == 4 ? 3 : 1) : bwd_occupancy<CT, D>())) void bwd_query(
    BwdParams P) {
  using TL = Tiles<CT, D>;
  using Frag = typename Mma<CT>::frag;
  constexpr int kNS = BID == BID_SOFTMAX ? 2 : 3;                // per-row statistics staged
  constexpr bool kPark = PARK && query_parks<CT, D>();
  static_assert(W == 4 || (W == 8 && kPark), "8-wave workgroups are the parked form");
  constexpr int kSteps = kTileK / Mma<CT>::kStep;
  constexpr int kFS = RowFrag<CT, D>::kSteps;
  __shared__ __attribute__((aligned(16))) CT k_s[2][kTileK * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT v_s[2][kTileK * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT kt_s[2][D * TL::kTStride];
  __shared__ __attribute__((aligned(16))) float rs_s[W][kNS * kTileQ];   // per wave: lse (r0), -dbs, r1
  __shared__ float g_s[W][kTileQ];
  // parked operands, lane-minor so that one fragment read is conflict-free:
  // each wave's dO' row fragments, and the identity of the transposes
  __shared__ __attribute__((aligned(16))) Frag do_park[kPark ? W : 1][kPark ? kFS : 1][64];
  __shared__ __attribute__((aligned(16))) Frag id_park[kPark ? kSteps : 1][64];

  const WorkItem item = xcd_work_item(P.kgroups, P.n, true, P.lpt != 0);    // heavy (late) row groups first
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int g = item.idx;
  // The plain wave index, deliberately: stated uniform (readfirstlane), it
  // turns the choice between the off-diagonal and the diagonal step into
  // scalar branches, and the compiler then copied the dq accumulators at
  // every step instead of keeping them in place.
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const float hf = static_cast<float>(h);
  const int qt = g * W + wave;
  const int64_t r0 = static_cast<int64_t>(qt) * kTileQ;
  const int64_t wg_last = min(static_cast<int64_t>(g * W + W) * kTileQ, P.T);
  const int nkt_wg = static_cast<int>((wg_last + kTileK - 1) / kTileK);
  const int nkt_w = r0 < P.T ? qt + 1 : 0;

  const CT* ks = static_cast<const CT*>(P.k) + slice * P.T * D;
  const CT* vs = static_cast<const CT*>(P.v) + slice * P.T * D;
  const CT* kts = static_cast<const CT*>(P.kt) + slice * D * P.t_pad;

  // this wave's rows in QS order: register i of half h <-> row r0 + 16 h + i
  RowFrag<CT, D> qf, dof;
  const int64_t my_row = r0 + qsig(l32);
  if (my_row < P.T) {
    load_row_frag<CT, D>(qf, static_cast<const CT*>(P.q) + (slice * P.T + my_row) * D + h * (D / 2));
    load_row_frag<CT, D>(dof, static_cast<const CT*>(P.dout) + (slice * P.T + my_row) * D + h * (D / 2));
  } else {
    zero_row_frag<CT, D>(qf);
    zero_row_frag<CT, D>(dof);
  }
  if (h == 0) {
    const int64_t r = r0 + l32;
    const bool ok = r < P.T;
    rs_s[wave][l32] = ok ? P.lse[slice * P.T + r] : (bid_log2<BID>() ? INFINITY : 0.f);
    rs_s[wave][kTileQ + l32] = ok ? -P.dbs[slice * P.T + r] : 0.f;
    if constexpr (kNS == 3) rs_s[wave][2 * kTileQ + l32] = ok ? P.rb1[slice * P.T + r] : 0.f;
  }
  Frag ident[kSteps];
  if constexpr (kPark) {
#pragma unroll
    for (int s = 0; s < kFS; ++s) do_park[wave][s][lane] = dof.f[s];
    if (wave == 0) {
#pragma unroll
      for (int s = 0; s < kSteps; ++s) id_park[s][lane] = ident_qs<CT>(l32, h, s);
    }
  } else {
#pragma unroll
    for (int s = 0; s < kSteps; ++s) ident[s] = ident_qs<CT>(l32, h, s);
  }
  auto ident_at = [&](int s) -> Frag {
    if constexpr (kPark) return id_park[s][lane];
    else return ident[s];
  };
  floatx16 dqa[kDTiles<D>];
#pragma unroll
  for (int t = 0; t < kDTiles<D>; ++t) dqa[t] = floatx16{};
  // ghat, parked form: this lane's share of the row sums of p dp, query
  // r0 + l32 over the keys that the transposed tile holds in this half.
  // Register form: ghat rides on the dq products as a ones column (column 0
  // of gacc).
  float gsum = 0.f;
  floatx16 gacc = floatx16{};
  const auto ones = ones_col_frag<CT>(l32);
  // demand and suffix checkpoints of this lane's key, loaded one key tile
  // ahead (steps past the wave's causal range never use them).  Parked form:
  // through resources that end at the row's last key (keys past T read 0; a
  // row tile past T has no checkpoint row and reads only zeros).  Register
  // form: guarded plain loads, as its tiles (measured faster there).
  const float* crow = P.carry + (slice * P.nb + qt) * P.T;
  const float* srow = P.sufk + (slice * P.nb + qt) * P.T;
  const int64_t ck_bytes = r0 < P.T ? P.T * 4 : 0;
  const auto crs = make_rsrc(crow, ck_bytes);
  const auto srs = make_rsrc(srow, ck_bytes);
  const uint32_t koff = static_cast<uint32_t>(rho(l32) * 4);
  auto ckpt_at = [&](int kt, bool suffix) -> float {
    if constexpr (kPark) {
      return buffer_load_f32(suffix ? srs : crs, static_cast<uint32_t>(kt * kTileK * 4) + koff, 0);
    } else {
      const int64_t key = static_cast<int64_t>(kt) * kTileK + rho(l32);
      return (kt < nkt_w && key < P.T) ? (suffix ? srow : crow)[key] : 0.f;
    }
  };

  auto step = [&](int kt, int buf, float cin, float sin, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const float* st = rs_s[wave];
    RowFrag<CT, D> kf, vf;
    lds_row_frag<CT, D>(kf, k_s[buf], rho(l32), h);
    lds_row_frag<CT, D>(vf, v_s[buf], rho(l32), h);
    float lz[16], ndb[16];
    lds_read16(st + kTileQ + 16 * h, ndb);
    // both score-shaped products first; ds = dO' V^T - dbs starts from -dbs
    // and runs under the p / demand chain
    const floatx16 sacc = mma_rows<CT, D>(qf, kf, floatx16{});
    floatx16 dov;
    if constexpr (kPark) {
      RowFrag<CT, D> dop;
#pragma unroll
      for (int s = 0; s < kFS; ++s) dop.f[s] = do_park[wave][s][lane];
      dov = mma_rows<CT, D>(dop, vf, as_x16(ndb));
    } else {
      dov = mma_rows<CT, D>(dof, vf, as_x16(ndb));
    }
    lds_read16(st + 16 * h, lz);
    float p[16], x[16], jac[16];
    if constexpr (BID == BID_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[i], P.c, -lz[i]));
    } else {
      float r1[16];
      lds_read16(st + 2 * kTileQ + 16 * h, r1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = bid_p<BID>(sacc[i], P.c, P.scale, lz[i], r1[i], P.lshift);
        jac[i] = bid_jac<BID>(p[i], sacc[i], P.scale, lz[i]);
      }
    }
    if constexpr (DIAG) {
      const int dk = rho(l32) - 16 * h;          // key - row(i) = dk - i on the diagonal tile
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dk > i) {
          p[i] = 0.f;
          jac[i] = 0.f;
        }
    }
    float ds[16];
    if constexpr (is_production<BID, SHARE>()) {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = p[i];
      scan_incl_qs(x, cin + kEps, hf);
      float sh[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = fast_rcp(x[i]);                   // inv
        sh[i] = p[i] * x[i];
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        ds[i] = dov[i] * sh[i];                  // ds sh
        x[i] = ds[i] * x[i];                     // g
      }
      scan_suffix_qs(x, sin, hf);                // x = G
#pragma unroll
      for (int i = 0; i < 16; ++i) ds[i] = fmaf(-p[i], x[i], ds[i]);   // p dp = ds sh - p G
    } else {
      // dp = ds inv - G (+ g for the exclusive share; ds with no share step)
      if constexpr (SHARE != SHARE_NONE) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = p[i];
        if constexpr (SHARE == SHARE_EXCL) scan_excl_qs(x, cin + kEps, hf);   // demand + eps
        else scan_incl_qs(x, cin + kEps, hf);                                // demand + p + eps
        float g[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float inv = fast_rcp(x[i]);
          ds[i] = dov[i] * inv;                  // ds inv
          g[i] = ds[i] * p[i] * inv;             // ds sh inv
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = g[i];
        scan_suffix_qs(x, sin, hf);              // x = G
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          ds[i] -= x[i];
          if constexpr (SHARE == SHARE_EXCL) ds[i] += g[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) ds[i] = dov[i];
      }
      // ds now holds dp; x takes p dp (the ghat operand)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = p[i] * ds[i];
        ds[i] = bid_log2<BID>() ? x[i] : jac[i] * ds[i];
      }
    }
    // transpose the dq operand (jac dp): queries in lanes, keys (natural order) in registers
    floatx16 xt = floatx16{};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) xt = Mma<CT>::mma_bexact(acc_frag<CT>(ds, s), ident_at(s), xt);
    float xv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = xt[i];
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto af = acc_frag<CT>(xv, s);
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
        dqa[t] = Mma<CT>::mma(af, lds_t_frag<CT, D>(kt_s[buf], 32 * t + l32, h, s), dqa[t]);
      if constexpr (!kPark && bid_log2<BID>()) gacc = Mma<CT>::mma_bexact(af, ones, gacc);
    }
    // the transposed values are exact copies of the dq operand (bf16 operands
    // in bf16 mode), so these are the row sums of what dq multiplies
    if constexpr (kPark && bid_log2<BID>()) gsum += sum16(xv);
    if constexpr (!bid_log2<BID>() && bid_normalized<BID>()) {
      // ghat needs the row sums of p dp, a different operand from jac dp here
      floatx16 yt = floatx16{};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) yt = Mma<CT>::mma_bexact(acc_frag<CT>(x, s), ident_at(s), yt);
      float yv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) yv[i] = yt[i];
      if constexpr (kPark) {
        gsum += sum16(yv);
      } else {
#pragma unroll
        for (int s = 0; s < kSteps; ++s) gacc = Mma<CT>::mma_bexact(acc_frag<CT>(yv, s), ones, gacc);
      }
    }
  };

  // buffer loads in the parked form; the register form skips the rows past
  // the end (both measured best for their form)
  // the tile loaders are laid out for kThreads threads: with 8 waves, waves
  // 0-3 stage the tiles that all 8 read (a wave-uniform condition)
  KTileLoader<CT, D, false, kPark ? kLoadBuffer : kLoadSkip> kl, vl;
  TTileLoader<CT, D, kPark ? kLoadBuffer : kLoadClamp> ktl;
  const bool stager = W == 4 || threadIdx.x < kThreads;
  auto fetch = [&](int kt) {
    if (!stager) return;
    const int64_t key0 = static_cast<int64_t>(kt) * kTileK;
    kl.load(ks, key0, P.T);
    vl.load(vs, key0, P.T);
    ktl.load(kts, key0);
  };
  auto stash = [&](int buf) {
    if (!stager) return;
    kl.store(k_s[buf]);
    vl.store(v_s[buf]);
    ktl.store(kt_s[buf]);
  };
  float cin_next = ckpt_at(0, false), sin_next = ckpt_at(0, true);
  fetch(0);
  stash(0);
  __syncthreads();
  auto iter = [&](int kt, int buf) __attribute__((always_inline)) {
    const float cin = cin_next, sin = sin_next;
    if (kt + 1 < nkt_wg) {
      fetch(kt + 1);
      cin_next = ckpt_at(kt + 1, false);
      sin_next = ckpt_at(kt + 1, true);
    }
    if (kt < qt && kt < nkt_w) step(kt, buf, cin, sin, std::false_type{});
    else if (kt == qt && kt < nkt_w) step(kt, buf, cin, sin, std::true_type{});
    if (kt + 1 < nkt_wg) stash(buf ^ 1);
    sync_lds();
  };
  double_buffered<!kPark>(0, nkt_wg, iter);      // the parked form has no registers to spare

  // ghat per query (the elementwise bids have no row normalisation and no ghat
  // term).  Parked: the two halves' partial sums of query r0 + l32.  Register
  // form: column 0 of gacc, register i of half h <-> row acc_row(i, h).
  if constexpr (kPark) {
    const HalfPair gp = halves(gsum);
    if (h == 0) g_s[wave][l32] = bid_normalized<BID>() ? gp.lo + gp.hi : 0.f;
  } else if (l32 == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) g_s[wave][acc_row(i, h)] = bid_normalized<BID>() ? gacc[i] : 0.f;
  }
  __syncthreads();
  if (h == 0 && r0 + l32 < P.T) P.ghat[slice * P.T + r0 + l32] = g_s[wave][l32];
  // the pk loads first (the dq stores could alias them for all the compiler knows)
  float pkv[16][kDTiles<D>];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = acc_row(i, h);
    const int64_t base = (slice * P.T + r0 + row) * D;
#pragma unroll
    for (int t = 0; t < kDTiles<D>; ++t) {
      const int d = 32 * t + l32;
      pkv[i][t] = (bid_normalized<BID>() && r0 + row < P.T && d < D) ? P.pk[base + d] : 0.f;
    }
  }
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = acc_row(i, h);
    if (r0 + row < P.T) {
      const float gr = g_s[wave][row];
      const int64_t base = (slice * P.T + r0 + row) * D;
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t) {
        const int d = 32 * t + l32;
        if (d < D) {
          const float corr = bid_normalized<BID>() ? gr * pkv[i][t] : 0.f;
          store_as(P.dq, base + d, P.gdt, dqa[t][i] * P.scale - corr);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// softmax-Jacobian correction of dk

template <typename CT, int D, int BID = BID_SOFTMAX>
__global__ __launch_bounds__(kThreads, (sizeof(CT) == 2 && D <= 64) ? 3 : 2) void bwd_dkcorr(BwdParams P) {
  using TL = Tiles<CT, D>;
  constexpr int kSplit = key_split<CT, D>();          // head-dim split as in bwd_key
  constexpr int kDH = D / kSplit;
  constexpr int kDT = kDTiles<kDH>;
  constexpr int kNS = BID == BID_SOFTMAX ? 1 : 3;                // per-row statistics staged
  __shared__ __attribute__((aligned(16))) CT q_s[2][kTileQ * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT qgt_s[2][kDH * TL::kTStride];
  __shared__ __attribute__((aligned(16))) float st_s[2][kNS * kTileQ];   // lse (r0), (unused), r1

  // Longest walks first (spread over the chip when the slices do not divide
  // over the XCDs) for short rows or uneven slice counts: -14% on this kernel
  // at B8 H16 T2048 and -11% at B1 H12 T16384.  Long rows over slices that
  // divide evenly keep contiguous ranges, slice by slice, whose Q tiles stay
  // in their XCD's L2 (about 1% faster at B1 H16 T16384).
  const bool lpt = P.lpt != 0 && (P.T <= 4096 || P.n % kXcds != 0);
  const WorkItem item = xcd_work_item(P.kgroups * kSplit, P.n, false, lpt, true);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int t0 = (item.idx % kSplit) * kDT;       // first 32-dim tile of the workgroup's head dims
  const int kb0 = (item.idx / kSplit) * 4;
  const int kb = kb0 + wave;
  const int64_t key = static_cast<int64_t>(kb) * kTileK + l32;
  const int nq = static_cast<int>((P.T + kTileQ - 1) / kTileQ);
  const bool active = static_cast<int64_t>(kb) * kTileK < P.T;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.T * D;
  const CT* qgts = static_cast<const CT*>(P.qgt) + slice * D * P.t_pad;
  const float* lse = P.lse + slice * P.T;

  RowFrag<CT, D> kf;
  if (key < P.T) load_row_frag<CT, D>(kf, static_cast<const CT*>(P.k) + (slice * P.T + key) * D + h * (D / 2));
  else zero_row_frag<CT, D>(kf);
  floatx16 dkc[kDT];
#pragma unroll
  for (int t = 0; t < kDT; ++t) dkc[t] = floatx16{};

  KTileLoader<CT, D, true> ql;            // row tile in query-split slot order
  TTileLoader<CT, kDH, kLoadBuffer, D> qtl;   // the workgroup's head dims of (ghat q)^T
  const int64_t t_off = static_cast<int64_t>(t0) * 32 * kTileK;
  RowStatsLoader<kNS, false> sl;
  if constexpr (!bid_log2<BID>()) sl.pad0 = 0.f;
  auto fetch = [&](int qt) {
    const int64_t row0 = static_cast<int64_t>(qt) * kTileQ;
    ql.load(qs, row0, P.T);
    qtl.load(qgts + t_off, row0);
    sl.load(lse, lse, BID == BID_SOFTMAX ? lse : P.rb1 + slice * P.T, row0, P.T);
  };
  auto stash = [&](int buf) {
    ql.store(q_s[buf]);
    qtl.store(qgt_s[buf]);
    sl.store(st_s[buf]);
  };
  constexpr int kSteps = kTileQ / Mma<CT>::kStep;

  auto step = [&](int buf, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    floatx16 sacc;                               // slot l32 holds row qsig(l32)
    if constexpr (kSplit > 1) {
      sacc = mma_rows_src<CT, D>(q_s[buf] + l32 * TL::kKStride + h * (D / 2), kf, floatx16{});
    } else {
      RowFrag<CT, D> qf;
      lds_row_frag<CT, D>(qf, q_s[buf], l32, h);
      sacc = mma_rows<CT, D>(qf, kf, floatx16{});
    }
    float lz[16], p[16];
    lds_read16(st_s[buf] + 16 * h, lz);
    if constexpr (BID == BID_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[i], P.c, -lz[i]));
    } else {
      // the correction runs on jac (p for the log2 bids)
      float r1[16];
      lds_read16(st_s[buf] + 2 * kTileQ + 16 * h, r1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = bid_p<BID>(sacc[i], P.c, P.scale, lz[i], r1[i], P.lshift);
        p[i] = bid_jac<BID>(pv, sacc[i], P.scale, lz[i]);
      }
    }
    if constexpr (DIAG) {
      const int dk = l32 - 16 * h;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dk > i) p[i] = 0.f;
    }
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto bfr = acc_frag<CT>(p, s);
#pragma unroll
      for (int t = 0; t < kDT; ++t)
        dkc[t] = Mma<CT>::mma(lds_tq_frag<CT, kDH>(qgt_s[buf], 32 * t + l32, h, s), bfr, dkc[t]);
    }
  };

  // elementwise bids have no ghat term: dk = scale * dk_main
  const int q_end = bid_normalized<BID>() ? nq : kb0;
  if (bid_normalized<BID>()) {
    fetch(kb0);
    stash(0);
  }
  __syncthreads();
  auto iter = [&](int qt, int buf) __attribute__((always_inline)) {
    if (qt + 1 < nq) fetch(qt + 1);
    if (active) {
      if (qt > kb) step(buf, std::false_type{});
      else if (qt == kb) step(buf, std::true_type{});
    }
    if (qt + 1 < nq) stash(buf ^ 1);
    sync_lds();
  };
  double_buffered<true>(kb0, q_end, iter);

  if (key < P.T) {
    // every dk_main load first (the dk stores could alias them for all the
    // compiler knows), four consecutive head dims per load and store
    const int64_t base = (slice * P.T + key) * D;
    floatx4 dm[kDT][4];
#pragma unroll
    for (int t = 0; t < kDT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * (t0 + t) + acc_row(4 * j, h);
        dm[t][j] = d < D ? *reinterpret_cast<const floatx4*>(P.dkm + base + d) : floatx4{};
      }
#pragma unroll
    for (int t = 0; t < kDT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * (t0 + t) + acc_row(4 * j, h);
        if (d < D) {
          floatx4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (dm[t][j][e] - dkc[t][4 * j + e]) * P.scale;
          store4_as(P.dk, base + d, P.gdt, v);
        }
      }
  }
}

// ---------------------------------------------------------------------------
// key-parallel reverse pass that also forms dq (bf16 operands, head_dim 64)
//
// bwd_key's walk, widened to 8 waves = 256 keys per workgroup, with the dq
// product done in the same walk instead of a second (row-parallel) sweep of
// the whole chain.  After each query tile every wave transposes its (p dp)
// tile with an identity MFMA (rows in lanes) and stages it in LDS as bf16;
// after the next step's chain the 8 waves then form the tile's dq contribution
// over the group's 256 keys, one 16 x 16 output block each
// (v_mfma_f32_16x16x32_bf16, K parked in LDS), and store it as a bf16
// partial per (key group, query tile), with the row sums of (p dp) (the
// ghat partials) in fp32.  bwd_dq_reduce adds the partials of every key
// group in a fixed order (deterministic, no atomics).
//
// Partials are stored compactly: key group g meets query tiles
// [8 g, nq), tile (g, qt) sits at keyq_tile_base(g, nq) + qt - 8 g (the
// key-group constants and this indexing live with the tile helpers: the
// forward's key pass uses them too).
//
// The bid / share variants run the same walk with bwd_key's variant chain:
// the per-row parameter r1 is staged with the statistics, the dk and dq
// operand is jac dp, the ratio bids' ghat partials are the row sums of p dp
// (a second transposed tile), and the elementwise bids have none.

// Storage type of the dq partials: bf16 by default; fp32 when built with
// -DDIL_KEYQ_F32_PARTIALS=1 (twice the bytes written and read back), the
// comparison build for the accuracy of the bf16 partials.
#ifndef DIL_KEYQ_F32_PARTIALS
#define DIL_KEYQ_F32_PARTIALS 0
#endif
using KqPart = std::conditional_t<DIL_KEYQ_F32_PARTIALS != 0, float, __bf16>;

template <int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
__global__ __launch_bounds__(kKqThreads, 2) void bwd_keyq(BwdParams P, KqPart* __restrict__ dqp,
                                                           float* __restrict__ ghp, int64_t ntiles) {
  static_assert(D == 64, "the dq-forming key pass is built for head_dim 64");
  using CT = __bf16;
  using TL = Tiles<CT, D>;
  constexpr int kNS = BID == BID_SOFTMAX ? 2 : 3;                // per-row statistics staged
  __shared__ __attribute__((aligned(16))) CT q_s[2][kTileQ * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT do_s[2][kTileQ * TL::kKStride];
  __shared__ __attribute__((aligned(16))) CT qt_s[2][D * TL::kTStride];
  __shared__ __attribute__((aligned(16))) CT dot_s[2][D * TL::kTStride];
  // lse (r0), -dbs, r1 of the tile's rows, then padding: every thread of the stash writes a slot
  __shared__ __attribute__((aligned(16))) float st_s[2][kKqThreads];
  __shared__ float cs_s[2][kKqKeys];                                   // demand entering the tile
  __shared__ __attribute__((aligned(16))) CT pd_s[2][kTileQ * kPdStride];   // (p dp), [row][key]
  __shared__ float gh_s[2][kKqWaves][kTileQ];                          // row sums of (p dp) per wave
  // B operand of the dq product: K of the group's keys, per d quarter and key
  // step (32 keys), lane-minor (one conflict-free 16-byte read per fragment)
  __shared__ __attribute__((aligned(16))) bf16x8 kpark[D / 16][kKqWaves][64];
  __shared__ __attribute__((aligned(16))) bf16x8 id_park[2][64];       // transpose identity

  // early keys (long walks) first, over the whole chip when the slices do not
  // divide over the XCDs (spread)
  const WorkItem item = xcd_work_item(P.kgroups, P.n, false, P.lpt != 0, true);
  if (!item.valid) return;
  const int64_t slice = item.slice;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const float hf = static_cast<float>(h);
  const int kg = item.idx;
  const int kb0 = kg * kKqWaves;                 // first key tile of the group
  const int kb = kb0 + wave;                     // key tile of this wave
  const int64_t key = static_cast<int64_t>(kb) * kTileK + l32;
  const int nq = static_cast<int>((P.T + kTileQ - 1) / kTileQ);
  const bool active = static_cast<int64_t>(kb) * kTileK < P.T;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.T * D;
  const CT* dos = static_cast<const CT*>(P.dout) + slice * P.T * D;
  const CT* qts = static_cast<const CT*>(P.qt) + slice * D * P.t_pad;
  const CT* dots = static_cast<const CT*>(P.dot) + slice * D * P.t_pad;
  const float* lse = P.lse + slice * P.T;
  const float* dbs = P.dbs + slice * P.T;

  // this wave's keys as B operands (lane <-> key)
  RowFrag<CT, D> kf, vf;
  if (key < P.T) {
    load_row_frag<CT, D>(kf, static_cast<const CT*>(P.k) + (slice * P.T + key) * D + h * (D / 2));
    load_row_frag<CT, D>(vf, static_cast<const CT*>(P.v) + (slice * P.T + key) * D + h * (D / 2));
  } else {
    zero_row_frag<CT, D>(kf);
    zero_row_frag<CT, D>(vf);
  }
  // park K of the group's keys for the dq product: fragment (d quarter u, key
  // step w, lane) holds K[32 (kb0 + w) + 8 (lane >> 4) + t][16 u + (lane & 15)],
  // t = 0..7: 16 contiguous bytes of the tile-major K^T copy (zero past the
  // slice's padded length, through the resource bound)
  {
    const CT* kts = static_cast<const CT*>(P.kt) + slice * D * P.t_pad;
    const int64_t first = static_cast<int64_t>(kb0) * kTileK * D;           // element offset of tile kb0
    const auto rs = make_rsrc(kts + first, (D * P.t_pad - first) * static_cast<int64_t>(sizeof(CT)));
#pragma unroll
    for (int u = 0; u < D / 16; ++u) {
      const int d = 16 * u + (lane & 15);
      const uint32_t off = static_cast<uint32_t>(((wave * D + d) * kTileK + 8 * (lane >> 4)) * sizeof(CT));
      kpark[u][wave][lane] = buffer_load16<bf16x8>(rs, off, 0);
    }
    if (wave == 0) {
#pragma unroll
      for (int s = 0; s < 2; ++s) id_park[s][lane] = ident_qs<CT>(l32, h, s);
    }
  }

  floatx16 dka[kDTiles<D>], dva[kDTiles<D>];
#pragma unroll
  for (int t = 0; t < kDTiles<D>; ++t) {
    dka[t] = floatx16{};
    dva[t] = floatx16{};
  }
  float sufk = 0.f;
  const bf16x8 ones8 = {__bf16(1.f), __bf16(1.f), __bf16(1.f), __bf16(1.f),
                        __bf16(1.f), __bf16(1.f), __bf16(1.f), __bf16(1.f)};

  // staging: waves 0-3 copy the Q row tile and its transpose, waves 4-7 dO'
  // and its transpose (one 16-byte chunk of each per thread); threads 0-63
  // the row statistics, threads 0-255 the demand checkpoints of the 256 keys
  const bool second = threadIdx.x >= 256;       // wave-uniform
  const int c256 = threadIdx.x & 255;
  const CT* rsrc = second ? dos : qs;
  const CT* tsrc = second ? dots : qts;
  bf16x8 rr = {}, tr = {};
  RowStatsLoader<kNS> sl;
  if constexpr (!bid_log2<BID>()) sl.pad0 = 0.f;
  const int64_t ck = static_cast<int64_t>(kb0) * kTileK + c256;
  const bool ck_ok = ck < P.T && !second;
  const float* ccol = P.carry + slice * P.nb * P.T + min(ck, P.T - 1);
  float cr = 0.f;
  // whole-slice resources, built once: the tile offset advances a 32-bit
  // per-lane offset (rows past T read as zeros through the resource bound)
  const auto rres = make_rsrc(rsrc, P.T * D * static_cast<int64_t>(sizeof(CT)));
  const auto tres = make_rsrc(tsrc, D * P.t_pad * static_cast<int64_t>(sizeof(CT)));
  auto fetch = [&](int qt) {
    const int64_t row0 = static_cast<int64_t>(qt) * kTileQ;
    const uint32_t off = static_cast<uint32_t>(qt) * static_cast<uint32_t>(kTileQ * D * sizeof(CT)) +
                         static_cast<uint32_t>(c256 * 16);
    rr = buffer_load16<bf16x8>(rres, off, 0);
    tr = buffer_load16<bf16x8>(tres, off, 0);
    sl.load(lse, dbs, BID == BID_SOFTMAX ? dbs : P.rb1 + slice * P.T, row0, P.T);
    cr = ccol[static_cast<int64_t>(qt) * P.T];
  };
  auto stash = [&](int buf) {
    {
      const int row = c256 / (D / 8), c = (c256 % (D / 8)) * 8;
      CT* dst = (second ? do_s[buf] : q_s[buf]) + qs_slot(row) * TL::kKStride + c;
      *reinterpret_cast<bf16x8*>(dst) = rr;
    }
    {
      const int d = c256 / (kTileQ / 8), c = (c256 % (kTileQ / 8)) * 8;
      CT* dst = (second ? dot_s[buf] : qt_s[buf]) + d * TL::kTStride + c;
      *reinterpret_cast<bf16x8*>(dst) = tr;
    }
    sl.store_all(st_s[buf]);
    if (!second) cs_s[buf][c256] = ck_ok ? cr : 0.f;
  };
  constexpr int kSteps = kTileQ / Mma<CT>::kStep;

  // (p dp) of this wave's keys for the tile, staged for the dq product from
  // the packed transposed tile: fragment s of half h holds keys acc_row(8 s +
  // t, h), two runs of 4 consecutive keys (16 s + 4 h, 16 s + 8 + 4 h)
  auto stage_pd = [&](int buf, const bf16x8 (&xf)[2]) {
    CT* dst = pd_s[buf] + l32 * kPdStride + wave * kTileK + 4 * h;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bf16x4 lo = {xf[s][0], xf[s][1], xf[s][2], xf[s][3]};
      const bf16x4 hi = {xf[s][4], xf[s][5], xf[s][6], xf[s][7]};
      *reinterpret_cast<bf16x4*>(dst + 16 * s) = lo;
      *reinterpret_cast<bf16x4*>(dst + 16 * s + 8) = hi;
    }
  };

  auto step = [&](int buf, auto diag_tag) {
    constexpr bool DIAG = decltype(diag_tag)::value;
    const float* st = st_s[buf];
    const float cin = cs_s[buf][wave * kTileK + l32];   // demand entering the tile
    RowFrag<CT, D> qf, dof;
    lds_row_frag<CT, D>(qf, q_s[buf], l32, h);      // slot l32 holds row qsig(l32)
    lds_row_frag<CT, D>(dof, do_s[buf], l32, h);
    float lz[16], ndb[16];
    lds_read16(st + kTileQ + 16 * h, ndb);
    const floatx16 sacc = mma_rows<CT, D>(qf, kf, floatx16{});
    const floatx16 dov = mma_rows<CT, D>(dof, vf, as_x16(ndb));
    lds_read16(st + 16 * h, lz);
    float p[16], x[16], sh[16], w[16];
    [[maybe_unused]] float jac[16];
    if constexpr (BID == BID_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < 16; ++i) p[i] = fast_exp2(fmaf(sacc[i], P.c, -lz[i]));
    } else {
      float r1[16];
      lds_read16(st + 2 * kTileQ + 16 * h, r1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = bid_p<BID>(sacc[i], P.c, P.scale, lz[i], r1[i], P.lshift);
        jac[i] = bid_jac<BID>(p[i], sacc[i], P.scale, lz[i]);
      }
    }
    if constexpr (DIAG) {
      const int dk = l32 - 16 * h;               // key - row(i) = dk - i on the diagonal tile
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (dk > i) {
          p[i] = 0.f;
          if constexpr (BID != BID_SOFTMAX) jac[i] = 0.f;
        }
    }
    if constexpr (SHARE != SHARE_NONE) {
#pragma unroll
      for (int i = 0; i < 16; ++i) x[i] = p[i];
      if constexpr (SHARE == SHARE_EXCL) scan_excl_qs(x, cin + kEps, hf);   // demand + eps
      else scan_incl_qs(x, cin + kEps, hf);                                // demand + p + eps
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        x[i] = fast_rcp(x[i]);                     // inv
        sh[i] = p[i] * x[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) sh[i] = p[i];
    }
    // dv^T += dO'^T sh  (keys in lanes; dO' carries the 1/(S+eps) of A)
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto bfr = acc_frag<CT>(sh, s);
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
        dva[t] = Mma<CT>::mma(lds_tq_frag<CT, D>(dot_s[buf], 32 * t + l32, h, s), bfr, dva[t]);
    }
    if constexpr (is_production<BID, SHARE>()) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        w[i] = dov[i] * sh[i];                     // ds sh
        x[i] = w[i] * x[i];                        // g = ds sh inv
      }
      sufk += scan_suffix_qs(x, sufk, hf);         // x = G
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] = fmaf(-p[i], x[i], w[i]);   // p dp = ds sh - p G
    } else {
      // dp = ds inv - G (+ g for the exclusive share; ds with no share step);
      // the MFMA operand is jac dp (jac = p for the log2 bids)
      if constexpr (SHARE != SHARE_NONE) {
        float g[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          w[i] = dov[i] * x[i];                    // ds inv
          g[i] = w[i] * sh[i];                     // ds sh inv
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = g[i];
        sufk += scan_suffix_qs(x, sufk, hf);       // x = G
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          w[i] -= x[i];
          if constexpr (SHARE == SHARE_EXCL) w[i] += g[i];
        }
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) w[i] = dov[i];
      }
      if constexpr (bid_ratio<BID>()) {
#pragma unroll
        for (int i = 0; i < 16; ++i) x[i] = p[i] * w[i];   // p dp, the ghat operand
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) w[i] *= bid_log2<BID>() ? p[i] : jac[i];
    }
    // dk_main^T += Q^T (jac dp), and the transposed (jac dp) for dq
    floatx16 xt = floatx16{};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const auto bfr = acc_frag<CT>(w, s);
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
        dka[t] = Mma<CT>::mma(lds_tq_frag<CT, D>(qt_s[buf], 32 * t + l32, h, s), bfr, dka[t]);
      xt = Mma<CT>::mma(bfr, id_park[s][lane], xt);
    }
    float xv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = xt[i];
    const bf16x8 xf[2] = {acc_frag<CT>(xv, 0), acc_frag<CT>(xv, 1)};
    stage_pd(buf, xf);
    // ghat partial of row l32 (the row sums of the bf16 operands dq
    // multiplies): all-ones A against the transposed tile, every register of
    // the result holds its lane's row sum
    floatx16 gs = floatx16{};
    if constexpr (bid_log2<BID>() && bid_normalized<BID>()) {
#pragma unroll
      for (int s = 0; s < 2; ++s) gs = Mma<CT>::mma(ones8, xf[s], gs);
    } else if constexpr (bid_normalized<BID>()) {
      // ghat needs the row sums of p dp, a different tile from the dq operand
      floatx16 yt = floatx16{};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) yt = Mma<CT>::mma(acc_frag<CT>(x, s), id_park[s][lane], yt);
      float yv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) yv[i] = yt[i];
#pragma unroll
      for (int s = 0; s < 2; ++s) gs = Mma<CT>::mma(ones8, acc_frag<CT>(yv, s), gs);
    }
    // (the elementwise bids have no row normalisation: their ghat is zero)
    if (h == 0) gh_s[buf][wave][l32] = gs[0];
  };
  // a wave whose keys all follow the tile's rows contributes nothing
  auto stage_zero = [&](int buf) {
    const bf16x8 z[2] = {bf16x8{}, bf16x8{}};
    stage_pd(buf, z);
    if (h == 0) gh_s[buf][wave][l32] = 0.f;
  };

  // dq contribution of the group's 256 keys to query tile qt: wave w forms
  // rows 16 (w & 1) + [0, 16) x head dims 16 (w >> 1) + [0, 16)
  const int rh = wave & 1, dq4 = wave >> 1;
  KqPart* dqp_s = dqp + slice * ntiles * (D * kTileQ);
  float* ghp_s = ghp + slice * ntiles * kTileQ;
  const int64_t gbase = keyq_tile_base(kg, nq) - static_cast<int64_t>(kKqTilesPerGroup) * kg;
  auto dq_product = [&](int qt, int buf) {
    if (qt < 0) return;
    floatx4 acc = floatx4{};
    const CT* arow = pd_s[buf] + (16 * rh + (lane & 15)) * kPdStride + 8 * (lane >> 4);
#pragma unroll
    for (int ks = 0; ks < kKqWaves; ++ks) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(arow + kTileK * ks);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, kpark[dq4][ks][lane], acc, 0, 0, 0);
    }
    // output: lane <-> head dim 16 dq4 + (lane & 15), register j <-> row 16 rh + 4 (lane >> 4) + j;
    // the partial tile is stored in 16 x 16 blocks (part_block_off)
    const int64_t tile = gbase + qt;
    KqPart* dst = dqp_s + tile * (D * kTileQ) + part_block_off(dq4, rh, lane);
    // streamed past the caches: the partials are read once, by bwd_dq_reduce
    if constexpr (std::is_same_v<KqPart, float>) {
      __builtin_nontemporal_store(acc, reinterpret_cast<floatx4*>(dst));
    } else {
      const floatx2 a = {acc[0], acc[1]}, b = {acc[2], acc[3]};
      const bf16x2 pa = __builtin_convertvector(a, bf16x2), pb = __builtin_convertvector(b, bf16x2);
      const bf16x4 v = {pa[0], pa[1], pb[0], pb[1]};
      __builtin_nontemporal_store(__builtin_bit_cast(floatx2, v), reinterpret_cast<floatx2*>(dst));
    }
    if (threadIdx.x < kTileQ) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < kKqWaves; ++w) s += gh_s[buf][w][threadIdx.x];
      __builtin_nontemporal_store(s, ghp_s + tile * kTileQ + threadIdx.x);
    }
  };

  const int late_dq = (threadIdx.x >> 8) ^ 1;     // wave-uniform: 1 for waves 0-3
  fetch(nq - 1);
  stash(0);
  __syncthreads();
  // the stash is unconditional (the last iteration stashes into the idle
  // buffer).  The dq product of tile qt + 1 (staged before the previous
  // barrier, in the other buffer) runs anywhere before this step's barrier,
  // which the stage of tile qt - 1 into that buffer follows.  Waves w and
  // w + 4 share a SIMD, and the barrier starts both in the same phase: waves
  // 4-7 run the dq product before their step, waves 0-3 after their stash,
  // so one wave's MFMA work issues under the other's VALU chain (-3% on this
  // kernel).  Both issue the partial store after the tile fetch, so the
  // stash, which waits for the fetch only, never waits for a store.
  auto iter = [&](int j, int buf) __attribute__((always_inline)) {
    const int qt = nq - 1 - j;                   // query tiles in reverse
    fetch(max(qt - 1, kb0));                     // the last step reloads its own tile, unused
    const int prev = j > 0 ? qt + 1 : -1;
    if (late_dq == 0) dq_product(prev, buf ^ 1);
    if (active && qt >= kb) {
      if (qt > kb) step(buf, std::false_type{});
      else step(buf, std::true_type{});
    } else {
      stage_zero(buf);
    }
    stash(buf ^ 1);
    if (late_dq != 0) dq_product(prev, buf ^ 1);
    sync_lds();
  };
  // unrolled by two for the production operator (253 VGPRs, no spills; 3%
  // faster); the variants' longer chains would spill, so they keep the loop
  double_buffered<is_production<BID, SHARE>()>(0, nq - kb0, iter);
  dq_product(kb0, (nq - kb0 - 1) & 1);          // the last tile, staged before the final barrier

  if (key < P.T) {
    // registers 4 j .. 4 j + 3 hold four consecutive head dims (acc_row)
    float* dkrow = P.dkm + (slice * P.T + key) * D;
    const int64_t dvrow = (slice * P.T + key) * D;
#pragma unroll
    for (int t = 0; t < kDTiles<D>; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d = 32 * t + acc_row(4 * j, h);
        if (d < D) {
          *reinterpret_cast<floatx4*>(dkrow + d) =
              floatx4{dka[t][4 * j], dka[t][4 * j + 1], dka[t][4 * j + 2], dka[t][4 * j + 3]};
          store4_as(P.dv, dvrow + d, P.gdt,
                    floatx4{dva[t][4 * j], dva[t][4 * j + 1], dva[t][4 * j + 2], dva[t][4 * j + 3]});
        }
      }
  }
}

// dq = scale * (sum over key groups of the dq partials) - ghat pk, ghat = the
// sum of the ghat partials, both in key-group order; and the (ghat * q)^T
// tiles of the dk correction.  Grid: (query tiles, slices from slice0), the
// tiles with the most key groups first.  Thread t sums elements [8 t, 8 t + 8)
// of the partial tiles (one head dim, 8 rows: part_dim / part_row).
template <int D, bool GHAT = true>
__global__ __launch_bounds__(kThreads) void bwd_dq_reduce(const KqPart* __restrict__ dqp,
                                                          const float* __restrict__ ghp, int64_t ntiles,
                                                          int64_t T, const float* __restrict__ pk,
                                                          const __bf16* __restrict__ qt, int64_t t_pad,
                                                          void* __restrict__ dq, int gdt, float scale,
                                                          __bf16* __restrict__ qgt, int64_t slice0) {
  static_assert(D * kTileQ == 8 * kThreads, "one 16-byte chunk of the partial tile per thread");
  __shared__ float sum_s[D][kTileQ + 1];
  __shared__ float g_s[kTileQ];
  const int64_t slice = slice0 + blockIdx.y;
  const int nq = static_cast<int>((T + kTileQ - 1) / kTileQ);
  const int tq = nq - 1 - static_cast<int>(blockIdx.x);
  const int ng = min(static_cast<int>(keyq_groups(T)) - 1, tq / kKqTilesPerGroup) + 1;
  const int t = threadIdx.x;
  const KqPart* base = dqp + slice * ntiles * (D * kTileQ) + 8 * t;
  // the partial sums are added in group order: deterministic
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto tile_of = [&](int g) { return keyq_tile_base(g, nq) + tq - kKqTilesPerGroup * g; };
  // a group's 8 values stay in their storage type until they are added (4
  // registers each for bf16: eight groups in flight keep the kernel at 8
  // waves per SIMD)
  using Raw = std::conditional_t<std::is_same_v<KqPart, float>, floatx8, bf16x8>;
  auto load_raw = [&](int g) -> Raw {
    const KqPart* p = base + tile_of(g) * (D * kTileQ);
    if constexpr (std::is_same_v<KqPart, float>) return __builtin_nontemporal_load(reinterpret_cast<const Raw*>(p));
    else return load_once(p);
  };
  // eight groups in flight; threads 0-31 load the same groups' ghat partials
  // beside them (both added in group order)
  const bool grow_t = GHAT && t < kTileQ;
  const float* gp = ghp + slice * ntiles * kTileQ + (grow_t ? t : 0);
  float s = 0.f;
  for (int g = 0; g < ng; g += 8) {
    Raw v[8];
    float r[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (g + u < ng) {
        v[u] = load_raw(g + u);
        if (grow_t) r[u] = load_once(gp + tile_of(g + u) * kTileQ);
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (g + u < ng) {
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += static_cast<float>(v[u][e]);
        if (grow_t) s += r[u];
      }
    }
  }
  {
    // the thread's 8 elements: one head dim, 8 consecutive rows of the tile
    const int pd = part_dim(8 * t), pr = part_row(8 * t);
#pragma unroll
    for (int e = 0; e < 8; ++e) sum_s[pd][pr + e] = acc[e];
  }
  const int d = t / (kTileQ / 8), r8 = (t % (kTileQ / 8)) * 8;
  if (grow_t) g_s[t] = s;
  __syncthreads();
  // (ghat * q)^T: thread t scales the [d][32 rows] chunk t of the tile-major Q^T copy (the
  // elementwise bids have no ghat and no dk correction)
  if constexpr (GHAT) {
    const int64_t off = slice * D * t_pad + tmajor_index(static_cast<int64_t>(tq) * kTileQ + r8, d, D);
    const bf16x8 qv = *reinterpret_cast<const bf16x8*>(qt + off);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = static_cast<float>(qv[e]) * g_s[r8 + e];
    store8<__bf16>(qgt + off, v);
  }
  // dq rows: thread t takes row t / 8, head dims 8 (t % 8) + [0, 8)
  const int row = t / (D / 8), d8 = (t % (D / 8)) * 8;
  const int64_t grow = static_cast<int64_t>(tq) * kTileQ + row;
  if (grow < T) {
    const int64_t o = (slice * T + grow) * D + d8;
    float v[8];
    if constexpr (GHAT) {
      const float gr = g_s[row];
      const floatx4* pk4 = reinterpret_cast<const floatx4*>(pk + o);
      const floatx4 pa = pk4[0], pb = pk4[1];
      const float pkv[8] = {pa[0], pa[1], pa[2], pa[3], pb[0], pb[1], pb[2], pb[3]};
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = sum_s[d8 + e][row] * scale - gr * pkv[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = sum_s[d8 + e][row] * scale;
    }
    store8_as(dq, o, gdt, v);
  }
}

// ---------------------------------------------------------------------------
// host side

struct BwdWorkspace {
  size_t lse, rb1, sinv, dbs, ghat, sufk, dkm, qt, kt, dot, qgt, qc, kc, vc, doc, total;
  size_t dqp, ghp;            // key-pass dq partials (alias sufk; the paths use one or the other)
};

// The dq-forming key pass serves bf16 operands at head_dim 64 while its
// partials (bf16 dq tiles + fp32 row sums: ~1 byte per causal score element)
// fit this budget; the row-parallel dq pass serves everything else.
constexpr int64_t kKeyqBudgetBytes = int64_t{24} << 30;

inline int64_t keyq_partial_bytes(int64_t n, int64_t T, int D) {
  return n * keyq_tiles(T) * (static_cast<int64_t>(D) * kTileQ * sizeof(KqPart) + kTileQ * 4);
}
inline bool keyq_eligible(int64_t n, int64_t T, int D, int prec) {
  // bwd_keyq reads the Q, dO' rows and their transposed copies through one
  // buffer resource per slice, which covers at most 2^31 - 1 bytes (the
  // budget already keeps T far below that: T^2 / 16 partials per slice)
  const int64_t slice_bytes = static_cast<int64_t>(D) * pad64(T) * 2;
  return prec == 2 && D == 64 && keyq_partial_bytes(n, T, D) <= kKeyqBudgetBytes && slice_bytes < (int64_t{1} << 31);
}

BwdWorkspace bwd_layout(int64_t n, int64_t T, int D, int dtype, int dout_dtype, int prec) {
  const size_t ct = prec == 2 ? 2 : 4;
  const int ctc = native_dtype(prec);
  const bool convert = dtype != ctc;
  const bool convert_do = dout_dtype != ctc;
  const int64_t nb = (T + kTileQ - 1) / kTileQ;
  const size_t rowf = align_up(4 * n * T);
  const size_t tsz = align_up(ct * n * D * pad64(T));
  const size_t rsz = align_up(ct * n * T * D);
  BwdWorkspace w{};
  w.lse = 0;
  w.rb1 = w.lse + rowf;
  w.sinv = w.rb1 + rowf;
  w.dbs = w.sinv + rowf;
  w.ghat = w.dbs + rowf;
  w.sufk = w.ghat + rowf;
  // the suffix checkpoints (row-parallel dq pass) and the key pass's dq
  // partials share one region
  size_t region = align_up(4 * n * nb * T);
  w.dqp = w.sufk;
  w.ghp = w.sufk;
  if (keyq_eligible(n, T, D, prec)) {
    const size_t dqb = align_up(static_cast<size_t>(n * keyq_tiles(T) * D * kTileQ * sizeof(KqPart)));
    w.ghp = w.dqp + dqb;
    region = std::max(region, dqb + align_up(static_cast<size_t>(n * keyq_tiles(T) * kTileQ * 4)));
  }
  w.dkm = w.sufk + region;
  w.qt = w.dkm + align_up(4 * n * T * D);
  w.kt = w.qt + tsz;
  w.dot = w.kt + tsz;
  w.qgt = w.dot + tsz;
  w.qc = w.qgt + tsz;
  w.kc = w.qc + (convert ? rsz : 0);
  w.vc = w.kc + (convert ? rsz : 0);
  w.doc = w.vc + (convert ? rsz : 0);
  w.total = w.doc + rsz;                      // dO' (dO scaled by sinv) is always built
  (void)convert_do;
  return w;
}

template <typename CT, int D, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
int launch_backward(const BackwardArgs& a) {
  // the workspace is sized for the worst case (dout converted), so that the
  // size query need not know dout's dtype
  const int ctc = kNativeDtype<CT>;
  const BwdWorkspace w = bwd_layout(a.n, a.T, D, a.dtype, ctc == DT_BF16 ? DT_F32 : DT_BF16, kOperandPrec<CT>);
  char* ws = static_cast<char*>(a.workspace);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const bool convert = a.dtype != ctc;
  const int64_t t_pad = pad64(a.T);
  const int64_t sn = a.T * D;

  CT* qt = reinterpret_cast<CT*>(ws + w.qt);
  CT* kt = reinterpret_cast<CT*>(ws + w.kt);
  CT* dot = reinterpret_cast<CT*>(ws + w.dot);
  CT* qgt = reinterpret_cast<CT*>(ws + w.qgt);
  CT* qc = convert ? reinterpret_cast<CT*>(ws + w.qc) : nullptr;
  CT* kc = convert ? reinterpret_cast<CT*>(ws + w.kc) : nullptr;
  CT* vc = convert ? reinterpret_cast<CT*>(ws + w.vc) : nullptr;
  CT* doc = reinterpret_cast<CT*>(ws + w.doc);

  const unsigned tiles64 = static_cast<unsigned>(t_pad / 64);
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    PrepJobs qkv{};
    qkv.job[0] = PrepJob{a.q, sn, qc, sn, qt, nullptr};
    qkv.job[1] = PrepJob{a.k, sn, kc, sn, kt, nullptr};
    qkv.job[2] = PrepJob{a.v, sn, vc, sn, nullptr, nullptr};
    DIL_TIMED("prep", st, (prep_kernel<CT, D><<<dim3(tiles64, ns, convert ? 3 : 2), kThreads, 0, st>>>(
                              qkv, a.dtype, a.T, D * t_pad, t_pad, s0)));
  });

  BwdParams P{};
  P.q = convert ? static_cast<const void*>(qc) : a.q;
  P.k = convert ? static_cast<const void*>(kc) : a.k;
  P.v = convert ? static_cast<const void*>(vc) : a.v;
  P.dout = doc;
  P.qt = qt;
  P.kt = kt;
  P.dot = dot;
  P.qgt = qgt;
  P.T = a.T;
  P.t_pad = t_pad;
  P.nb = (a.T + kTileQ - 1) / kTileQ;
  P.scale = 1.f / sqrtf(static_cast<float>(D));
  P.c = kLog2e * P.scale;
  float* lse = reinterpret_cast<float*>(ws + w.lse);
  float* sinv = reinterpret_cast<float*>(ws + w.sinv);
  float* dbs = reinterpret_cast<float*>(ws + w.dbs);
  P.lse = lse;
  P.rb1 = reinterpret_cast<float*>(ws + w.rb1);
  P.lshift = log2f(a.var.shift);
  P.sinv = sinv;
  P.dbs = dbs;
  P.ghat = reinterpret_cast<float*>(ws + w.ghat);
  P.carry = a.carry;
  P.sufk = reinterpret_cast<float*>(ws + w.sufk);
  P.dkm = reinterpret_cast<float*>(ws + w.dkm);
  P.pk = a.pk;
  P.dq = a.dq;
  P.dk = a.dk;
  P.dv = a.dv;
  P.gdt = a.grad_dtype;
  P.lpt = longest_first_for(a.n, a.T);

  // row statistics and dO' = dO / (S + eps), row-major and transposed
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    DIL_TIMED("bwd_rows", st, (bwd_rows<CT, D, BID><<<dim3(tiles64, ns), kThreads, 0, st>>>(
                                  a.dout, a.dout_dtype, a.out, a.rmax, a.rden, a.ssum, lse, sinv, dbs,
                                  reinterpret_cast<float*>(ws + w.rb1), a.T, t_pad, doc, dot, s0)));
  });
  const int nkt = static_cast<int>((a.T + kTileK - 1) / kTileK);
  P.n = a.n;
  if constexpr (std::is_same_v<CT, __bf16> && D == 64) {
    if (keyq_eligible(a.n, a.T, D, kOperandPrec<CT>)) {
      // one key pass forms dv, dk_main and the dq partials; the reduction
      // finishes dq and writes the (ghat q)^T tiles of the dk correction
      KqPart* dqp = reinterpret_cast<KqPart*>(ws + w.dqp);
      float* ghp = reinterpret_cast<float*>(ws + w.ghp);
      const int64_t ntiles = keyq_tiles(a.T);
      P.kgroups = static_cast<int>(keyq_groups(a.T));
      const dim3 gkq(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(P.kgroups) * a.n)));
      DIL_TIMED("bwd_keyq", st, (bwd_keyq<D, BID, SHARE><<<gkq, kKqThreads, 0, st>>>(P, dqp, ghp, ntiles)));
      const unsigned nq = static_cast<unsigned>((a.T + kTileQ - 1) / kTileQ);
      slice_batches(a.n, [&](int64_t s0, unsigned ns) {
        constexpr bool kGhat = bid_normalized<BID>();   // the elementwise bids have no ghat
        DIL_TIMED("bwd_dq_reduce", st,
                  (bwd_dq_reduce<D, kGhat><<<dim3(nq, ns), kThreads, 0, st>>>(dqp, ghp, ntiles, a.T, a.pk, qt, t_pad,
                                                                             a.dq, a.grad_dtype, P.scale, qgt, s0)));
      });
      P.kgroups = (nkt + 3) / 4;
      const dim3 gkey(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(P.kgroups) * key_split<CT, D>() * a.n)));
      DIL_TIMED("bwd_dkcorr", st, (bwd_dkcorr<CT, D, BID><<<gkey, kThreads, 0, st>>>(P)));
      return static_cast<int>(hipGetLastError());
    }
  }
  P.kgroups = (nkt + 3) / 4;
  // bwd_key and bwd_dkcorr: key groups x head-dim parts x slices
  const dim3 gkeys(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(P.kgroups) * key_split<CT, D>() * a.n)));
  DIL_TIMED("bwd_key", st, (bwd_key<CT, D, BID, SHARE><<<gkeys, kThreads, 0, st>>>(P)));
  constexpr bool kParked = query_parks<CT, D>() && is_production<BID, SHARE>();
  constexpr int kQW = kParked ? query_waves<CT, D>() : 4;     // row tiles (waves) per workgroup
  {
    const int kgroups_key = P.kgroups;
    P.kgroups = (nkt + kQW - 1) / kQW;
    const dim3 gq(static_cast<unsigned>(xcd_grid(static_cast<int64_t>(P.kgroups) * a.n)));
    DIL_TIMED("bwd_query", st, (bwd_query<CT, D, BID, SHARE, kParked, kQW><<<gq, 64 * kQW, 0, st>>>(P)));
    P.kgroups = kgroups_key;
  }
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    DIL_TIMED("prep", st,
              prep_ghat_q<CT, D><<<dim3(static_cast<unsigned>(t_pad / 32), ns), kThreads, 0, st>>>(
                  qt, P.ghat, a.T, t_pad, qgt, s0));
  });
  DIL_TIMED("bwd_dkcorr", st, (bwd_dkcorr<CT, D, BID><<<gkeys, kThreads, 0, st>>>(P)));
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace dil
