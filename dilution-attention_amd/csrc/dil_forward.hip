// Forward of the dilution-attention operator (plain forward and chunked
// prefill share these kernels).
//
// Reference behaviour: dilution_attention_forward,
// /root/reference/src/dilution/kernels.py:328-455, whose row-parallel
// decomposition (K1 :137-198 -> block scan :251-264 -> K2 :267-315) this
// follows in structure; the kernels are written for gfx950 MFMA layouts:
//
//   prep       convert q/k to the MFMA operand type when needed; write V^T
//              (and K^T for pk) tiles, zero-padded to a multiple of 64 keys.
//   fwd_stats  one workgroup = 4 waves = 4 tiles of 32 query rows; key tiles
//              of 32 staged in LDS.  Sweep 1 computes S^T = K Q^T so each lane
//              owns one query row: online row max / 2^-sum (log2 domain), and
//              optionally pk^T = K^T p^T with online rescaling.  Sweep 2
//              recomputes S = Q K^T (each lane owns one key column) and writes
//              the per-32-row-block column sums of p.
//   fwd_scan   exclusive scan of the block sums over blocks (fp64 running sum)
//              -> carry checkpoints; inclusive total -> committed_total.
//   fwd_out    S = Q K^T with keys in lanes: p, the in-tile column scan on
//              registers plus the checkpoint, share = p / (demand + p + eps),
//              row sums; the share tile is transposed by one MFMA against an
//              identity operand so that share @ V runs on MFMA with queries in
//              lanes.  out = (share @ V) / (rowsum + eps).
//
// Nothing T x T is stored: scratch is the (n, C/32, Tk) fp32 checkpoint array.
#include "dil_common.hpp"
#include "dil_internal.hpp"
#include "dil_tiles.hpp"

namespace dil {

namespace {

struct FwdParams {
  const void* q;          // CT rows (n, C, D), slice stride q_sn
  int64_t q_sn;
  const void* k;          // CT rows (n, >= Tk, D), slice stride k_sn
  int64_t k_sn;
  const void* vt;         // CT (n, D, Tk_pad)
  const void* kt;         // CT (n, D, Tk_pad) or null
  int64_t t_sn, tk_pad;
  int64_t C, Tk, q0, nb;
  float c;                // log2(e) / sqrt(D)
  float scale;            // 1 / sqrt(D)
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
};

// ---------------------------------------------------------------------------
// row statistics + block column sums

template <typename CT, int D, bool PK>
__global__ __launch_bounds__(kThreads) void fwd_stats(FwdParams P) {
  using T = Tiles<CT, D>;
  __shared__ __attribute__((aligned(16))) CT ktile[2][kTileK * T::kKStride];
  __shared__ __attribute__((aligned(16))) CT kttile[PK ? 2 : 1][PK ? D * T::kTStride : 1];
  __shared__ float lse_s[4][kTileQ];

  const int64_t slice = blockIdx.y;
  const int g = gridDim.x - 1 - blockIdx.x;            // heavy (late) row groups first
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int64_t r0 = (static_cast<int64_t>(g) * 4 + wave) * kTileQ;   // first row of this wave (chunk-relative)
  const int64_t qa0 = P.q0 + r0;                                     // absolute index of that row
  const int64_t wg_last = min(P.q0 + (static_cast<int64_t>(g) * 4 + 4) * kTileQ, P.Tk);  // keys < wg_last
  const int nkt_wg = static_cast<int>((wg_last + kTileK - 1) / kTileK);
  const int64_t w_last = min(qa0 + kTileQ, P.Tk);
  const int nkt_w = r0 < P.C ? static_cast<int>((w_last + kTileK - 1) / kTileK) : 0;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  const CT* ks = static_cast<const CT*>(P.k) + slice * P.k_sn;
  const CT* kts = PK ? static_cast<const CT*>(P.kt) + slice * P.t_sn : nullptr;

  RowFrag<CT, D> qf;
  if (r0 + l32 < P.C) load_row_frag<CT, D>(qf, qs + (r0 + l32) * D + h * (D / 2));
  else zero_row_frag<CT, D>(qf);
  const int64_t my_q = qa0 + l32;   // query owned by this lane in sweep 1

  KTileLoader<CT, D> kl;
  TTileLoader<CT, D> tl;

  // ---- sweep 1: S^T = K Q^T, one query per lane ----
  float mraw = -INFINITY, lsum = 0.f;
  floatx16 pka[PK ? kDTiles<D> : 1];
  if constexpr (PK) {
#pragma unroll
    for (int t = 0; t < kDTiles<D>; ++t) pka[t] = floatx16{};
  }
  kl.load(ks, 0, P.Tk);
  if constexpr (PK) tl.load(kts, P.tk_pad, 0);
  kl.store(ktile[0]);
  if constexpr (PK) tl.store(kttile[0]);
  __syncthreads();
  for (int kt = 0; kt < nkt_wg; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt_wg) {
      kl.load(ks, static_cast<int64_t>(kt + 1) * kTileK, P.Tk);
      if constexpr (PK) tl.load(kts, P.tk_pad, static_cast<int64_t>(kt + 1) * kTileK);
    }
    if (kt < nkt_w) {
      RowFrag<CT, D> kf;
      lds_row_frag<CT, D>(kf, ktile[buf], rho(l32), h);
      floatx16 acc = mma_rows<CT, D>(kf, qf, floatx16{});
      float a[16];
      const int64_t key0 = static_cast<int64_t>(kt) * kTileK;
      const bool diag = key0 + kTileK - 1 > qa0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        a[i] = acc[i];
        if (diag && key0 + perm_row(i, h) > my_q) a[i] = -INFINITY;
      }
      float tmax = a[0];
#pragma unroll
      for (int i = 1; i < 16; ++i) tmax = fmaxf(tmax, a[i]);
      float mnew = fmaxf(mraw, tmax);
      if constexpr (PK) mnew = fmaxf(mnew, partner32(mnew));
      const float msafe = (mnew == -INFINITY) ? 0.f : mnew;
      const float alpha = (mraw == -INFINITY) ? 0.f : fast_exp2((mraw - msafe) * P.c);
      const float mc = msafe * P.c;
      float e[16];
      float add = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        e[i] = fast_exp2(fmaf(a[i], P.c, -mc));
        add += e[i];
      }
      lsum = fmaf(lsum, alpha, add);
      if constexpr (PK) {
        // rescale only when some lane's maximum moved
        if (__any(alpha != 1.f)) {
#pragma unroll
          for (int t = 0; t < kDTiles<D>; ++t) pka[t] *= alpha;
        }
#pragma unroll
        for (int s = 0; s < kTileK / Mma<CT>::kStep; ++s) {
          const auto bfr = acc_frag<CT>(e, s);
#pragma unroll
          for (int t = 0; t < kDTiles<D>; ++t)
            pka[t] = Mma<CT>::mma(lds_t_frag<CT, D>(kttile[buf], 32 * t + l32, h, s), bfr, pka[t]);
        }
      }
      mraw = mnew;
    }
    if (kt + 1 < nkt_wg) {
      kl.store(ktile[buf ^ 1]);
      if constexpr (PK) tl.store(kttile[buf ^ 1]);
    }
    __syncthreads();
  }
  // combine the two lane halves (different keys, same query)
  const float pm = partner32(mraw), pl = partner32(lsum);
  const float mtot = fmaxf(mraw, pm);
  const float mts = (mtot == -INFINITY) ? 0.f : mtot;
  const float ltot = (mraw == -INFINITY ? 0.f : lsum * fast_exp2((mraw - mts) * P.c)) +
                     (pm == -INFINITY ? 0.f : pl * fast_exp2((pm - mts) * P.c));
  const bool row_ok = r0 + l32 < P.C;
  const float rmax_v = mtot * P.c;
  if (h == 0 && row_ok) {
    P.rmax[slice * P.C + r0 + l32] = rmax_v;
    P.rden[slice * P.C + r0 + l32] = ltot;
  }
  if (h == 0) lse_s[wave][l32] = row_ok ? rmax_v + __log2f(ltot) : INFINITY;
  if constexpr (PK) {
    // halves share the running max, so pka holds the full sum over keys
    if (row_ok) {
      const float f = P.scale / ltot;
      float* dst = P.pk + (slice * P.C + r0 + l32) * D;
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * t + acc_row(i, h) < D) dst[32 * t + acc_row(i, h)] = pka[t][i] * f;
    }
  }
  __syncthreads();

  // ---- sweep 2: S = Q K^T, one key per lane: block column sums of p ----
  float lse[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) lse[i] = lse_s[wave][acc_row(i, h)];
  float* sblk = P.carry + (slice * P.nb + r0 / kTileQ) * P.Tk;
  kl.load(ks, 0, P.Tk);
  kl.store(ktile[0]);
  __syncthreads();
  for (int kt = 0; kt < nkt_wg; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt_wg) kl.load(ks, static_cast<int64_t>(kt + 1) * kTileK, P.Tk);
    if (kt < nkt_w) {
      RowFrag<CT, D> kf;
      lds_row_frag<CT, D>(kf, ktile[buf], l32, h);
      floatx16 acc = mma_rows<CT, D>(qf, kf, floatx16{});
      const int64_t key = static_cast<int64_t>(kt) * kTileK + l32;
      const bool diag = static_cast<int64_t>(kt) * kTileK + kTileK - 1 > qa0;
      float cs = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float p = fast_exp2(fmaf(acc[i], P.c, -lse[i]));
        if (diag && key > qa0 + acc_row(i, h)) p = 0.f;
        cs += p;
      }
      cs += partner32(cs);
      if (h == 0 && key < P.Tk) sblk[key] = cs;
    }
    if (kt + 1 < nkt_wg) kl.store(ktile[buf ^ 1]);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// exclusive scan of block column sums -> carry checkpoints, totals

__global__ __launch_bounds__(256) void fwd_scan(float* __restrict__ carry, int64_t nb, int64_t Tk,
                                                int64_t q0, int64_t C,
                                                const float* __restrict__ demand_in, int64_t din_sn,
                                                float* __restrict__ total, int64_t tot_sn) {
  const int64_t slice = blockIdx.y;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (j >= Tk) return;
  double run = (demand_in != nullptr && j < q0) ? static_cast<double>(demand_in[slice * din_sn + j]) : 0.0;
  float* col = carry + slice * nb * Tk + j;
  for (int64_t b = 0; b < nb; ++b) {
    // block b covers rows [q0 + 32 b, q0 + 32 b + 32); keys at or beyond its
    // end were not written by fwd_stats (their sum is zero by causality)
    const bool written = j < q0 + 32 * (b + 1) && 32 * b < C;
    const float s = written ? col[b * Tk] : 0.f;
    col[b * Tk] = static_cast<float>(run);
    run += static_cast<double>(s);
  }
  total[slice * tot_sn + j] = static_cast<float>(run);
}

// ---------------------------------------------------------------------------
// output pass

template <typename CT, int D>
__global__ __launch_bounds__(kThreads) void fwd_out(FwdParams P) {
  using T = Tiles<CT, D>;
  __shared__ __attribute__((aligned(16))) CT ktile[2][kTileK * T::kKStride];
  __shared__ __attribute__((aligned(16))) CT vttile[2][D * T::kTStride];
  __shared__ float ssum_s[4][kTileQ];

  const int64_t slice = blockIdx.y;
  const int g = gridDim.x - 1 - blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
  const int64_t r0 = (static_cast<int64_t>(g) * 4 + wave) * kTileQ;
  const int64_t qa0 = P.q0 + r0;
  const int64_t wg_last = min(P.q0 + (static_cast<int64_t>(g) * 4 + 4) * kTileQ, P.Tk);
  const int nkt_wg = static_cast<int>((wg_last + kTileK - 1) / kTileK);
  const int64_t w_last = min(qa0 + kTileQ, P.Tk);
  const int nkt_w = r0 < P.C ? static_cast<int>((w_last + kTileK - 1) / kTileK) : 0;

  const CT* qs = static_cast<const CT*>(P.q) + slice * P.q_sn;
  const CT* ks = static_cast<const CT*>(P.k) + slice * P.k_sn;
  const CT* vts = static_cast<const CT*>(P.vt) + slice * P.t_sn;

  // Q rows loaded rho-permuted: accumulator register i of half h <-> row perm_row(i, h)
  RowFrag<CT, D> qf;
  const int64_t my_row = r0 + rho(l32);
  if (my_row < P.C) load_row_frag<CT, D>(qf, qs + my_row * D + h * (D / 2));
  else zero_row_frag<CT, D>(qf);

  float lse[16], rsum[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t r = r0 + perm_row(i, h);
    lse[i] = (r < P.C) ? P.rmax[slice * P.C + r] + __log2f(P.rden[slice * P.C + r]) : INFINITY;
    rsum[i] = 0.f;
  }
  constexpr int kSteps = kTileK / Mma<CT>::kStep;
  typename Mma<CT>::frag ident[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) ident[s] = ident_frag<CT>(l32, h, s);
  floatx16 o[kDTiles<D>];
#pragma unroll
  for (int t = 0; t < kDTiles<D>; ++t) o[t] = floatx16{};
  const float* crow = P.carry + (slice * P.nb + r0 / kTileQ) * P.Tk;

  KTileLoader<CT, D> kl;
  TTileLoader<CT, D> vl;
  kl.load(ks, 0, P.Tk);
  vl.load(vts, P.tk_pad, 0);
  kl.store(ktile[0]);
  vl.store(vttile[0]);
  __syncthreads();
  for (int kt = 0; kt < nkt_wg; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nkt_wg) {
      kl.load(ks, static_cast<int64_t>(kt + 1) * kTileK, P.Tk);
      vl.load(vts, P.tk_pad, static_cast<int64_t>(kt + 1) * kTileK);
    }
    if (kt < nkt_w) {
      const int64_t key0 = static_cast<int64_t>(kt) * kTileK;
      const int64_t key = key0 + rho(l32);          // key owned by this lane
      RowFrag<CT, D> kf;
      lds_row_frag<CT, D>(kf, ktile[buf], rho(l32), h);
      floatx16 acc = mma_rows<CT, D>(qf, kf, floatx16{});
      const bool diag = key0 + kTileK - 1 > qa0;
      float p[16], x[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        p[i] = fast_exp2(fmaf(acc[i], P.c, -lse[i]));
        if (diag && key > qa0 + perm_row(i, h)) p[i] = 0.f;
        x[i] = p[i];
      }
      const float cin = (key < P.Tk) ? crow[key] : 0.f;
      column_scan_inclusive(x, cin + kEps, h);
      float sh[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        sh[i] = p[i] * fast_rcp(x[i]);
        rsum[i] += sh[i];
      }
      // transpose the share tile: X[key][query] with queries in lanes
      floatx16 xt = floatx16{};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) xt = Mma<CT>::mma(acc_frag<CT>(sh, s), ident[s], xt);
      float xv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) xv[i] = xt[i];
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const auto af = acc_frag<CT>(xv, s);
#pragma unroll
        for (int t = 0; t < kDTiles<D>; ++t)
          o[t] = Mma<CT>::mma(af, lds_t_frag<CT, D>(vttile[buf], 32 * t + l32, h, s), o[t]);
      }
    }
    if (kt + 1 < nkt_wg) {
      kl.store(ktile[buf ^ 1]);
      vl.store(vttile[buf ^ 1]);
    }
    __syncthreads();
  }

  // row sums: reduce over the 32 lanes of each half (keys), then publish
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float v = rsum[i];
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) v += __shfl_xor(v, off, 64);
    rsum[i] = v;
  }
  if (l32 == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) ssum_s[wave][perm_row(i, h)] = rsum[i];
  }
  __syncthreads();
  if (h == 0 && r0 + l32 < P.C) P.ssum[slice * P.C + r0 + l32] = ssum_s[wave][l32];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int row = acc_row(i, h);
    if (r0 + row < P.C) {
      const float inv = 1.f / (ssum_s[wave][row] + kEps);
      float* dst = P.out + slice * P.o_sn + (r0 + row) * D;
#pragma unroll
      for (int t = 0; t < kDTiles<D>; ++t)
        if (32 * t + l32 < D) dst[32 * t + l32] = o[t][i] * inv;
    }
  }
}

// ---------------------------------------------------------------------------
// host side

struct FwdWorkspace {
  size_t vt, kt, qc, kc, total;
};

FwdWorkspace fwd_layout(int64_t n, int64_t C, int64_t Tk, int D, int dtype, int lowp, int want_pk) {
  const size_t ct = lowp ? 2 : 4;
  const bool convert = lowp ? dtype != DT_BF16 : dtype != DT_F32;
  FwdWorkspace w{};
  const size_t tsz = align_up(ct * n * D * pad64(Tk));
  w.vt = 0;
  w.kt = w.vt + tsz;
  w.qc = w.kt + (want_pk ? tsz : 0);
  w.kc = w.qc + (convert ? align_up(ct * n * C * D) : 0);
  w.total = w.kc + (convert ? align_up(ct * n * Tk * D) : 0);
  return w;
}

template <typename CT, int D>
int launch_forward(const ForwardArgs& a) {
  const FwdWorkspace w = fwd_layout(a.n, a.C, a.Tk, D, a.dtype, a.lowp, a.pk != nullptr);
  char* ws = static_cast<char*>(a.workspace);
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  const bool convert = sizeof(CT) == 2 ? a.dtype != DT_BF16 : a.dtype != DT_F32;
  const int64_t tk_pad = pad64(a.Tk);
  const unsigned n = static_cast<unsigned>(a.n);

  CT* vt = reinterpret_cast<CT*>(ws + w.vt);
  CT* kt = a.pk ? reinterpret_cast<CT*>(ws + w.kt) : nullptr;
  CT* qc = convert ? reinterpret_cast<CT*>(ws + w.qc) : nullptr;
  CT* kc = convert ? reinterpret_cast<CT*>(ws + w.kc) : nullptr;

  // operands in the compute type; V^T (and K^T) tiles
  const dim3 gk(static_cast<unsigned>(tk_pad / 64), n);
  DIL_TIMED("prep", st,
            prep_kernel<CT, D><<<gk, kThreads, 0, st>>>(a.v, a.kv_sn, a.dtype, a.Tk, nullptr, 0, vt,
                                                        D * tk_pad, tk_pad));
  if (convert || kt != nullptr)
    DIL_TIMED("prep", st,
              prep_kernel<CT, D><<<gk, kThreads, 0, st>>>(a.k, a.kv_sn, a.dtype, a.Tk, kc, a.Tk * D,
                                                          kt, D * tk_pad, tk_pad));
  if (convert) {
    const dim3 gq(static_cast<unsigned>(pad64(a.C) / 64), n);
    DIL_TIMED("prep", st,
              prep_kernel<CT, D><<<gq, kThreads, 0, st>>>(a.q, a.q_sn, a.dtype, a.C, qc, a.C * D,
                                                          nullptr, 0, 0));
  }

  FwdParams P{};
  P.q = convert ? static_cast<const void*>(qc) : a.q;
  P.q_sn = convert ? a.C * D : a.q_sn;
  P.k = convert ? static_cast<const void*>(kc) : a.k;
  P.k_sn = convert ? a.Tk * D : a.kv_sn;
  P.vt = vt;
  P.kt = kt;
  P.t_sn = D * tk_pad;
  P.tk_pad = tk_pad;
  P.C = a.C;
  P.Tk = a.Tk;
  P.q0 = a.q0;
  P.nb = (a.C + kTileQ - 1) / kTileQ;
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

  const dim3 grid(static_cast<unsigned>((a.C + 4 * kTileQ - 1) / (4 * kTileQ)), n);
  if (a.pk) DIL_TIMED("fwd_stats", st, fwd_stats<CT, D, true><<<grid, kThreads, 0, st>>>(P));
  else DIL_TIMED("fwd_stats", st, fwd_stats<CT, D, false><<<grid, kThreads, 0, st>>>(P));
  DIL_TIMED("fwd_scan", st,
            fwd_scan<<<dim3(static_cast<unsigned>((a.Tk + 255) / 256), n), 256, 0, st>>>(
                a.carry, P.nb, a.Tk, a.q0, a.C, a.demand_in, a.din_sn, a.total, a.tot_sn));
  DIL_TIMED("fwd_out", st, fwd_out<CT, D><<<grid, kThreads, 0, st>>>(P));
  return static_cast<int>(hipGetLastError());
}

template <int D>
int dispatch_forward(const ForwardArgs& a) {
  return a.lowp ? launch_forward<__bf16, D>(a) : launch_forward<float, D>(a);
}

}  // namespace

int64_t forward_workspace_bytes(int64_t n, int64_t C, int64_t Tk, int head_dim, int dtype, int lowp,
                                int want_pk) {
  return static_cast<int64_t>(fwd_layout(n, C, Tk, head_dim, dtype, lowp, want_pk).total);
}

int forward(const ForwardArgs& a) {
  switch (a.head_dim) {
    case 16: return dispatch_forward<16>(a);
    case 32: return dispatch_forward<32>(a);
    case 64: return dispatch_forward<64>(a);
    case 128: return dispatch_forward<128>(a);
    default: return kErrHeadDim;
  }
}

}  // namespace dil
