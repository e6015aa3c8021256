// Few-row projections of the LM's decode step (include/dilution_hip.h:
// dil_rows_linear): out[m, n] for m < rows <= 8 rows of bf16 activations
// against an nn.Linear weight W (N, K), with the decode step's neighbours
// folded in:
//   mode 0  out = x W^T
//   mode 1  out = resid + x W^T
//   mode 2  out = rmsnorm(x) W^T,                  rmsnorm(x) = x / rms(x) * g
//   mode 3  out = silu(r W1^T) * (r W2^T),         r = rmsnorm(x)
// Every intermediate is rounded to bf16 where the separate torch ops round
// it (the RMSNorm output, x / rms(x) * g in fp32 rounded once as torch's GPU
// rms_norm does; each product; silu; the sum of the residual add), so the
// result follows the unfused bf16 layer within the accumulation order of the
// dot products.
//
// At rows = batch = 8 the product is bound by streaming W once from HBM (2 B
// per weight against 16 FLOPs); a library GEMM tiled for large M reads it at
// a fraction of HBM speed.  Here one workgroup of 4 waves takes 8 W rows per
// wave (KSPLIT = 1) or 8 W rows split over the waves' K ranges (KSPLIT = 4),
// so that a small N still fills the GPU.  Within a wave, 8 lanes cover one W
// row: lane s reads 16 bytes at k = 8 (s + 8 j), the 8 lanes one 128-byte
// segment, and multiplies them with the staged activations (an LDS broadcast:
// the 8 rows of a wave read the same 8 chunks) on v_dot2_f32_bf16 with fp32
// accumulation; three xor shuffles add the 8 lanes of a row.
#include <hip/hip_runtime.h>

#include "../../include/dilution_hip.h"
#include "dil_common.hpp"
#include "dil_internal.hpp"

namespace dil {
namespace {

constexpr int kLinRows = 8;            // activation rows (the decode batch)
constexpr int kLinThreads = 256;
constexpr int kLinMaxK = 4096;

__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float c) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    c = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{a[2 * j], a[2 * j + 1]}, bf16x2{b[2 * j], b[2 * j + 1]}, c, false);
  return c;
}

__device__ __forceinline__ float round_bf16(float v) { return static_cast<float>(static_cast<__bf16>(v)); }

template <int MODE, int KSPLIT>
__global__ __launch_bounds__(kLinThreads) void rows_linear(const __bf16* __restrict__ x, const __bf16* __restrict__ w1,
                                                           const __bf16* __restrict__ w2, const __bf16* __restrict__ g,
                                                           const __bf16* __restrict__ resid, __bf16* __restrict__ out,
                                                           int rows, int64_t N, int K, float eps) {
  constexpr bool kNorm = MODE >= 2;
  constexpr bool kPair = MODE == 3;
  constexpr int kRowsPerWave = 8;
  constexpr int kRowsPerWg = kRowsPerWave * 4 / KSPLIT;
  __shared__ __attribute__((aligned(16))) bf16x8 xs[kLinRows][kLinMaxK / 8];
  __shared__ float red[4][kRowsPerWave][kLinRows][kPair ? 2 : 1];

  const int t = threadIdx.x;
  const int nchunk = K / 8;
  // ---- stage the activations (thread t: row t / 32, chunks t % 32 + 32 i) ----
  {
    const int m = t >> 5, c0 = t & 31;
    const int per = nchunk / 32;                 // K is a multiple of 256
    float ss = 0.f;
    for (int i = 0; i < per; ++i) {
      const int c = c0 + 32 * i;
      bf16x8 v = {};
      if (m < rows) v = *reinterpret_cast<const bf16x8*>(x + static_cast<int64_t>(m) * K + 8 * c);
      xs[m][c] = v;
      if constexpr (kNorm) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(static_cast<float>(v[e]), static_cast<float>(v[e]), ss);
      }
    }
    if constexpr (kNorm) {
      // the 32 threads of a row (one half of a wave) add their sums
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) ss += __shfl_xor(ss, o, 32);
      const float inv = rsqrtf(ss / static_cast<float>(K) + eps);
      for (int i = 0; i < per; ++i) {
        const int c = c0 + 32 * i;
        const bf16x8 v = xs[m][c];
        const bf16x8 gw = *reinterpret_cast<const bf16x8*>(g + 8 * c);
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = static_cast<float>(v[e]) * inv * static_cast<float>(gw[e]);
        xs[m][c] = Mma<__bf16>::pack(r);
      }
    }
  }
  __syncthreads();

  // ---- the products ----
  const int wave = t >> 6, lane = t & 63, r = lane >> 3, s = lane & 7;
  const int row_in_wg = KSPLIT == 1 ? wave * kRowsPerWave + r : r;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kRowsPerWg + row_in_wg;
  const int64_t nc = n < N ? n : N - 1;          // rows past N read a valid row, never stored
  const int kc_per = nchunk / KSPLIT;            // chunks of this wave's K range
  const int kc0 = KSPLIT == 1 ? 0 : wave * kc_per;
  const __bf16* w1r = w1 + nc * K;
  const __bf16* w2r = kPair ? w2 + nc * K : nullptr;
  float a1[kLinRows], a2[kLinRows];
#pragma unroll
  for (int m = 0; m < kLinRows; ++m) a1[m] = a2[m] = 0.f;
  constexpr int kUnroll = 4;
  const int iters = kc_per / 8;                  // chunks per lane
  for (int j0 = 0; j0 < iters; j0 += kUnroll) {
    bf16x8 wa[kUnroll], wb[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = kc0 + s + 8 * (j0 + u);
      if (j0 + u < iters) {
        wa[u] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(w1r + 8 * c));
        if constexpr (kPair) wb[u] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(w2r + 8 * c));
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (j0 + u < iters) {
        const int c = kc0 + s + 8 * (j0 + u);
#pragma unroll
        for (int m = 0; m < kLinRows; ++m) {
          const bf16x8 xv = xs[m][c];
          a1[m] = dot8(wa[u], xv, a1[m]);
          if constexpr (kPair) a2[m] = dot8(wb[u], xv, a2[m]);
        }
      }
    }
  }
  // the 8 lanes of a row
#pragma unroll
  for (int m = 0; m < kLinRows; ++m) {
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
      a1[m] += __shfl_xor(a1[m], o, 8);
      if constexpr (kPair) a2[m] += __shfl_xor(a2[m], o, 8);
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
    out[static_cast<int64_t>(m) * N + nn] = static_cast<__bf16>(v);
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

template <int MODE>
int launch_rows_linear(const __bf16* x, const __bf16* w1, const __bf16* w2, const __bf16* g, const __bf16* resid,
                       __bf16* out, int rows, int64_t N, int K, float eps, hipStream_t st) {
  // waves split K when one row per lane group would leave the GPU short of
  // workgroups (N below 8192 rows: 256 CUs x 32 rows)
  if (N < 8192) {
    const dim3 grid(static_cast<unsigned>((N + 7) / 8));
    rows_linear<MODE, 4><<<grid, kLinThreads, 0, st>>>(x, w1, w2, g, resid, out, rows, N, K, eps);
  } else {
    const dim3 grid(static_cast<unsigned>((N + 31) / 32));
    rows_linear<MODE, 1><<<grid, kLinThreads, 0, st>>>(x, w1, w2, g, resid, out, rows, N, K, eps);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace dil

extern "C" int dil_rows_linear(const void* x, const void* w1, const void* w2, const void* g, const void* resid,
                               void* out, int64_t rows, int64_t n, int64_t k, int mode, int dtype, float eps,
                               void* stream) {
  using dil::kErrShape;
  if (dtype != dil::DT_BF16) return dil::kErrDtype;
  if (mode < 0 || mode > 3) return kErrShape;
  if (rows < 1 || rows > dil::kLinRows || n < 1 || k < 256 || k > dil::kLinMaxK || k % 256 != 0) return kErrShape;
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
  switch (mode) {
    case 0: return dil::launch_rows_linear<0>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, st);
    case 1: return dil::launch_rows_linear<1>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, st);
    case 2: return dil::launch_rows_linear<2>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, st);
    default: return dil::launch_rows_linear<3>(xb, w1b, w2b, gb, rb, ob, r, n, kk, eps, st);
  }
}
