// Few-row projections of the LM's decode step (include/dilution_hip.h:
// dil_rows_linear, dil_rows_linear_qkv): out[m, n] for m < rows <= 8 rows of
// bf16 activations against an nn.Linear weight W (N, K), with the decode
// step's neighbours folded in:
//   mode 0  out = x W^T
//   mode 1  out = resid + x W^T
//   mode 2  out = rmsnorm(x) W^T,                  rmsnorm(x) = x / rms(x) * g
//   mode 3  out = silu(r W1^T) * (r W2^T),         r = rmsnorm(x)
//   mode 4  mode 2 with W = [Wq; Wk; Wv] (N = 3 H D): the q part to out
//           (rows, H D), the k and v parts stored as the new row `pos` of the
//           (rows, H, capacity, D) key and value caches
// Every intermediate is rounded to bf16 where the separate torch ops round
// it (the RMSNorm output, x / rms(x) * g in fp32 rounded once as torch's GPU
// rms_norm does; each product; silu; the sum of the residual add), so the
// result follows the unfused bf16 layer within the accumulation order of the
// dot products.
//
// At rows = batch = 8 the product is bound by streaming W once from HBM (2 B
// per weight against 16 FLOPs); a library GEMM tiled for large M reads it at
// a fraction of HBM speed.  Here one workgroup of 4 waves takes 8 W rows per
// wave (KSPLIT = 1), or 8 or 4 W rows split over the waves' K ranges
// (KSPLIT = 4), so that a small N still fills the GPU.  Within a wave, LPR = 8
// (or 16) lanes cover one W row: lane s reads 16 bytes at k = 8 (s + LPR j),
// the LPR lanes one 128-byte (256-byte) segment, and multiplies them with the
// staged activations (an LDS broadcast: the W rows of a wave read the same
// chunks) on v_dot2_f32_bf16 with fp32 accumulation; xor shuffles add the LPR
// lanes of a row.
//
// The matrices are small (2-100 MB), so a launch is latency-bound.  A thread
// loads its activation chunks into registers, then issues its first 8 or 16
// weight loads, and stages the activations in LDS while the weights are in
// flight (loads complete in issue order, so waiting for the activations never
// waits for the weights).  The activation buffer is sized for K (16 KB at K
// up to 1024) so that several workgroups share a CU.
#include <hip/hip_runtime.h>

#include "../../include/dilution_hip.h"
#include "dil_common.hpp"
#include "dil_internal.hpp"

namespace dil {
namespace {

constexpr int kLinRows = 8;            // activation rows (the decode batch)
constexpr int kLinThreads = 256;
constexpr int kLinMaxK = 4096;

// Where mode 4 puts its three parts.
struct QkvDst {
  __bf16* kc;                          // (rows, heads, capacity, head_dim)
  __bf16* vc;
  int64_t capacity;
  const int64_t* pos_dev;              // the new row's position on the device, or null
  int64_t pos;                         // ... on the host when pos_dev is null
  int heads, head_dim;
};

__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float c) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    c = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{a[2 * j], a[2 * j + 1]}, bf16x2{b[2 * j], b[2 * j + 1]}, c, false);
  return c;
}

__device__ __forceinline__ float round_bf16(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

template <int MODE, int KSPLIT, int KCAP, int LPR>
__global__ __launch_bounds__(kLinThreads) void rows_linear(const __bf16* __restrict__ x, const __bf16* __restrict__ w1,
                                                           const __bf16* __restrict__ w2, const __bf16* __restrict__ g,
                                                           const __bf16* __restrict__ resid, __bf16* __restrict__ out,
                                                           int rows, int64_t N, int K, float eps, QkvDst qkv) {
  constexpr bool kNorm = MODE >= 2;
  constexpr bool kPair = MODE == 3;
  constexpr int kRowsPerWave = 64 / LPR;         // W rows of a wave, LPR lanes each
  constexpr int kRowsPerWg = kRowsPerWave * 4 / KSPLIT;
  // weight loads in flight per lane (8 where a lane has two matrices, or where
  // KSPLIT = 1 keeps the registers low enough for five waves per SIMD)
  constexpr int U = kPair || KSPLIT == 1 ? 8 : 16;
  constexpr int kPerMax = KCAP / 256;            // activation chunks staged per thread
  constexpr bool kGEarly = kNorm && KCAP <= 1024;
  __shared__ __attribute__((aligned(16))) bf16x8 xs[kLinRows][KCAP / 8];
  __shared__ float red[4][kRowsPerWave][kLinRows][kPair ? 2 : 1];

  const int t = threadIdx.x;
  const int nchunk = K / 8;

  // ---- the activations (and norm weights) first: thread t takes row t / 32,
  //      chunks t % 32 + 32 i, into registers ----
  const int xm = t >> 5, xc0 = t & 31;
  const int per = nchunk / 32;                   // K is a multiple of 256
  bf16x8 xv[kPerMax], gv[kGEarly ? kPerMax : 1];
#pragma unroll
  for (int i = 0; i < kPerMax; ++i) {
    xv[i] = bf16x8{};
    if (i < per && xm < rows) xv[i] = *reinterpret_cast<const bf16x8*>(x + static_cast<int64_t>(xm) * K + 8 * (xc0 + 32 * i));
    if constexpr (kGEarly) {
      if (i < per) gv[i] = *reinterpret_cast<const bf16x8*>(g + 8 * (xc0 + 32 * i));
    }
  }

  // ---- then the first weight loads, in flight while the activations are staged ----
  const int wave = t >> 6, lane = t & 63, r = lane / LPR, s = lane % LPR;
  const int row_in_wg = KSPLIT == 1 ? wave * kRowsPerWave + r : r;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + row_in_wg;
  const int64_t nc = n < N ? n : N - 1;          // rows past N read a valid row, never stored
  const int kc_per = nchunk / KSPLIT;            // chunks of this wave's K range
  const int kc0 = KSPLIT == 1 ? 0 : wave * kc_per;
  const __bf16* w1r = w1 + nc * K;
  const __bf16* w2r = kPair ? w2 + nc * K : nullptr;
  const int iters = kc_per / LPR;                // chunks per lane
  bf16x8 wa[U], wb[U];
  auto load = [&](int j0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = kc0 + s + LPR * (j0 + u);
      if (j0 + u < iters) {
        wa[u] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(w1r + 8 * c));
        if constexpr (kPair) wb[u] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(w2r + 8 * c));
      }
    }
  };
  load(0);

  // ---- stage the activations, normalised in the norm modes ----
  if constexpr (kNorm) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kPerMax; ++i) {
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(static_cast<float>(xv[i][e]), static_cast<float>(xv[i][e]), ss);
    }
    // the 32 threads of a row (one half of a wave) add their sums
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) ss += __shfl_xor(ss, o, 32);
    const float inv = rsqrtf(ss / static_cast<float>(K) + eps);
#pragma unroll
    for (int i = 0; i < kPerMax; ++i) {
      if (i < per) {
        bf16x8 gw;
        if constexpr (kGEarly) gw = gv[i];
        else gw = *reinterpret_cast<const bf16x8*>(g + 8 * (xc0 + 32 * i));
        float rr[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) rr[e] = static_cast<float>(xv[i][e]) * inv * static_cast<float>(gw[e]);
        xs[xm][xc0 + 32 * i] = Mma<__bf16>::pack(rr);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPerMax; ++i)
      if (i < per) xs[xm][xc0 + 32 * i] = xv[i];
  }
  __syncthreads();

  // ---- the products ----
  float a1[kLinRows], a2[kLinRows];
#pragma unroll
  for (int m = 0; m < kLinRows; ++m) a1[m] = a2[m] = 0.f;
  for (int j0 = 0; j0 < iters; j0 += U) {
    if (j0 > 0) load(j0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (j0 + u < iters) {
        const int c = kc0 + s + LPR * (j0 + u);
#pragma unroll
        for (int m = 0; m < kLinRows; ++m) {
          const bf16x8 xq = xs[m][c];
          a1[m] = dot8(wa[u], xq, a1[m]);
          if constexpr (kPair) a2[m] = dot8(wb[u], xq, a2[m]);
        }
      }
    }
  }
  // the LPR lanes of a W row
#pragma unroll
  for (int m = 0; m < kLinRows; ++m) {
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) {
      a1[m] += __shfl_xor(a1[m], o, LPR);
      if constexpr (kPair) a2[m] += __shfl_xor(a2[m], o, LPR);
    }
  }
  auto finish = [&](int m, int64_t nn, float v1, float v2) {
    float v;
    if constexpr (MODE == 3) {
      const float gt = round_bf16(v1), up = round_bf16(v2);
      const float act = round_bf16(gt / (1.f + expf(-gt)));
      v = act * up;
    } else if constexpr (MODE == 1) {
      v = round_bf16(v1) + static_cast<float>(resid[static_cast<int64_t>(m) * N + nn]);
    } else {
      v = v1;
    }
    if constexpr (MODE == 4) {
      const int64_t dm = N / 3;
      const int part = static_cast<int>(nn / dm);
      const int64_t c = nn - part * dm;
      if (part == 0) {
        out[static_cast<int64_t>(m) * dm + c] = static_cast<__bf16>(v);
      } else {
        const int64_t p = qkv.pos_dev != nullptr ? *qkv.pos_dev : qkv.pos;
        if (p >= 0 && p < qkv.capacity) {        // a position outside the cache is never written
          const int64_t h = c / qkv.head_dim, e = c - h * qkv.head_dim;
          __bf16* cache = part == 1 ? qkv.kc : qkv.vc;
          cache[((static_cast<int64_t>(m) * qkv.heads + h) * qkv.capacity + p) * qkv.head_dim + e] =
              static_cast<__bf16>(v);
        }
      }
    } else {
      out[static_cast<int64_t>(m) * N + nn] = static_cast<__bf16>(v);
    }
  };
  if constexpr (KSPLIT == 1) {
    if (s == 0 && n < N) {
      for (int m = 0; m < rows; ++m) finish(m, n, a1[m], a2[m]);
    }
  } else {
    // the waves' K ranges, added in wave order
    if (s == 0) {
#pragma unroll
      for (int m = 0; m < kLinRows; ++m) {
        red[wave][r][m][0] = a1[m];
        if constexpr (kPair) red[wave][r][m][kPair ? 1 : 0] = a2[m];
      }
    }
    __syncthreads();
    if (t < kRowsPerWave * kLinRows) {
      const int rr = t / kLinRows, m = t % kLinRows;
      const int64_t nn = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + rr;
      if (m < rows && nn < N) {
        float v1 = 0.f, v2 = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          v1 += red[w][rr][m][0];
          if constexpr (kPair) v2 += red[w][rr][m][kPair ? 1 : 0];
        }
        finish(m, nn, v1, v2);
      }
    }
  }
}

template <int MODE, int KSPLIT, int LPR>
void launch_kcap(const __bf16* x, const __bf16* w1, const __bf16* w2, const __bf16* g, const __bf16* resid,
                 __bf16* out, int rows, int64_t N, int K, float eps, const QkvDst& qkv, hipStream_t st) {
  constexpr int kRowsPerWg = 64 / LPR * 4 / KSPLIT;
  const dim3 grid(static_cast<unsigned>((N + kRowsPerWg - 1) / kRowsPerWg));
  if (K <= 1024)
    rows_linear<MODE, KSPLIT, 1024, LPR><<<grid, kLinThreads, 0, st>>>(x, w1, w2, g, resid, out, rows, N, K, eps,
                                                                        qkv);
  else
    rows_linear<MODE, KSPLIT, kLinMaxK, LPR><<<grid, kLinThreads, 0, st>>>(x, w1, w2, g, resid, out, rows, N, K,
                                                                            eps, qkv);
}

template <int MODE>
int launch_rows_linear(const __bf16* x, const __bf16* w1, const __bf16* w2, const __bf16* g, const __bf16* resid,
                       __bf16* out, int rows, int64_t N, int K, float eps, const QkvDst& qkv, hipStream_t st) {
  // Enough workgroups to cover 256 CUs: from N = 8192 up, 32 W rows per
  // workgroup (8 per wave); below, the 4 waves split K over 8 W rows; below
  // N = 2048, over 4 W rows of 16 lanes each (K a multiple of 512, so that
  // every lane has whole chunks).
  if (N >= 8192)
    launch_kcap<MODE, 1, 8>(x, w1, w2, g, resid, out, rows, N, K, eps, qkv, st);
  else if (N >= 2048 || K % 512 != 0)
    launch_kcap<MODE, 4, 8>(x, w1, w2, g, resid, out, rows, N, K, eps, qkv, st);
  else
    launch_kcap<MODE, 4, 16>(x, w1, w2, g, resid, out, rows, N, K, eps, qkv, st);
  return static_cast<int>(hipGetLastError());
}

// Greedy selection over the head's logits: per row, the index of the largest
// of the first `limit` values, as torch.argmax picks it (a NaN counts as the
// largest value, and among equal values the smallest index wins).  One
// 1024-thread workgroup per row; 16-byte loads when the rows are aligned.
constexpr int kArgThreads = 1024;

__device__ __forceinline__ bool arg_better(float a, int ia, float b, int ib) {
  const bool an = a != a, bn = b != b;
  if (an != bn) return an;
  if (!an && a != b) return a > b;
  return ia < ib;
}

template <bool VEC>
__global__ __launch_bounds__(kArgThreads) void rows_argmax(const __bf16* __restrict__ logits, int64_t stride,
                                                           int limit, int64_t* __restrict__ out) {
  const __bf16* p = logits + static_cast<int64_t>(blockIdx.x) * stride;
  const int t = threadIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  if constexpr (VEC) {
    const int nvec = limit / 8;
    constexpr int kU = 8;
    for (int c0 = t; c0 < nvec; c0 += kU * kArgThreads) {
      bf16x8 v[kU];
#pragma unroll
      for (int u = 0; u < kU; ++u)
        if (c0 + u * kArgThreads < nvec) v[u] = reinterpret_cast<const bf16x8*>(p)[c0 + u * kArgThreads];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int c = c0 + u * kArgThreads;
        if (c < nvec) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float x = static_cast<float>(v[u][e]);
            if (arg_better(x, 8 * c + e, best, bi)) { best = x; bi = 8 * c + e; }
          }
        }
      }
    }
    for (int i = 8 * nvec + t; i < limit; i += kArgThreads) {
      const float x = static_cast<float>(p[i]);
      if (arg_better(x, i, best, bi)) { best = x; bi = i; }
    }
  } else {
    for (int i = t; i < limit; i += kArgThreads) {
      const float x = static_cast<float>(p[i]);
      if (arg_better(x, i, best, bi)) { best = x; bi = i; }
    }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (arg_better(ob, oi, best, bi)) { best = ob; bi = oi; }
  }
  __shared__ float sb[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  if ((t & 63) == 0) { sb[t >> 6] = best; si[t >> 6] = bi; }
  __syncthreads();
  if (t == 0) {
    for (int w = 1; w < kArgThreads / 64; ++w)
      if (arg_better(sb[w], si[w], best, bi)) { best = sb[w]; bi = si[w]; }
    out[blockIdx.x] = bi;
  }
}

bool rows_k_ok(int64_t rows, int64_t k) {
  return rows >= 1 && rows <= kLinRows && k >= 256 && k <= kLinMaxK && k % 256 == 0;
}

}  // namespace
}  // namespace dil

extern "C" int dil_rows_linear(const void* x, const void* w1, const void* w2, const void* g, const void* resid,
                               void* out, int64_t rows, int64_t n, int64_t k, int mode, int dtype, float eps,
                               void* stream) {
  using dil::kErrShape;
  if (dtype != dil::DT_BF16) return dil::kErrDtype;
  if (mode < 0 || mode > 3) return kErrShape;
  if (!dil::rows_k_ok(rows, k) || n < 1) return kErrShape;
  if (x == nullptr || w1 == nullptr || out == nullptr) return kErrShape;
  if (mode == 1 && resid == nullptr) return kErrShape;
  if (mode >= 2 && g == nullptr) return kErrShape;
  if (mode == 3 && w2 == nullptr) return kErrShape;
  if (!(eps >= 0.f)) return kErrShape;
  const auto* xb = static_cast<const __bf16*>(x);
  const auto* w1b = static_cast<const __bf16*>(w1);
  const auto* w2b = static_cast<const __bf16*>(w2);
  const auto* gb = static_cast<const __bf16*>(g);
  const auto* rb = static_cast<const __bf16*>(resid);
  auto* ob = static_cast<__bf16*>(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int r = static_cast<int>(rows), kk = static_cast<int>(k);
  const dil::QkvDst none{};
  switch (mode) {
    case 0: return dil::launch_rows_linear<0>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, none, st);
    case 1: return dil::launch_rows_linear<1>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, none, st);
    case 2: return dil::launch_rows_linear<2>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, none, st);
    default: return dil::launch_rows_linear<3>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, none, st);
  }
}

extern "C" int dil_rows_linear_qkv(const void* x, const void* w, const void* g, void* q_out, void* k_cache,
                                   void* v_cache, int64_t rows, int64_t heads, int64_t head_dim, int64_t capacity,
                                   const int64_t* pos_dev, int64_t pos, int64_t k, int dtype, float eps,
                                   void* stream) {
  using dil::kErrShape;
  if (dtype != dil::DT_BF16) return dil::kErrDtype;
  if (!dil::rows_k_ok(rows, k) || heads < 1 || head_dim < 1 || capacity < 1) return kErrShape;
  if (heads * head_dim > (int64_t{1} << 24)) return kErrShape;
  if (x == nullptr || w == nullptr || g == nullptr || q_out == nullptr || k_cache == nullptr || v_cache == nullptr)
    return kErrShape;
  if (pos_dev == nullptr && (pos < 0 || pos >= capacity)) return kErrShape;
  if (!(eps >= 0.f)) return kErrShape;
  const dil::QkvDst dst{static_cast<__bf16*>(k_cache), static_cast<__bf16*>(v_cache), capacity, pos_dev, pos,
                        static_cast<int>(heads), static_cast<int>(head_dim)};
  return dil::launch_rows_linear<4>(static_cast<const __bf16*>(x), static_cast<const __bf16*>(w), nullptr,
                                    static_cast<const __bf16*>(g), nullptr, static_cast<__bf16*>(q_out),
                                    static_cast<int>(rows), 3 * heads * head_dim, static_cast<int>(k), eps, dst,
                                    static_cast<hipStream_t>(stream));
}

extern "C" int dil_rows_argmax(const void* logits, int64_t rows, int64_t row_stride, int64_t limit, void* out,
                               int dtype, void* stream) {
  if (dtype != dil::DT_BF16) return dil::kErrDtype;
  if (logits == nullptr || out == nullptr || rows < 1 || rows > 65535 || limit < 1 || limit > 0x7fffffff ||
      row_stride < limit)
    return dil::kErrShape;
  const auto* lb = static_cast<const __bf16*>(logits);
  auto* ob = static_cast<int64_t*>(out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = row_stride % 8 == 0 && reinterpret_cast<uintptr_t>(logits) % 16 == 0;
  const dim3 grid(static_cast<unsigned>(rows));
  if (vec)
    dil::rows_argmax<true><<<grid, dil::kArgThreads, 0, st>>>(lb, row_stride, static_cast<int>(limit), ob);
  else
    dil::rows_argmax<false><<<grid, dil::kArgThreads, 0, st>>>(lb, row_stride, static_cast<int>(limit), ob);
  return static_cast<int>(hipGetLastError());
}
