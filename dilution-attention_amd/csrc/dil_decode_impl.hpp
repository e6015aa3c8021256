// Cached decode step: one new query row per (batch, head) slice against
// `length` cached keys, with the per-key fp32 demand vector advanced in place.
//
// Reference behaviour: /root/reference/src/dilution/kernels.py:937-991
// (_dilution_decode) and :994-1038 (dilution_decode_step).  The reference runs
// one program per slice; here the keys are split into chunks so the grid fills
// 256 CUs, in three launches:
//
//   dec_stats  (chunks x n): a_j = q.k_j * scale*log2e -> fp32 scratch AFF,
//                            chunk-local (max, sum 2^(a-max))
//   dec_apply  (chunks x n): combine the chunk statistics -> lse; for every key
//                            p = 2^(a-lse), share = p / (committed + p + eps),
//                            chunk partials sum(share), sum(share * v);
//                            committed += p stored in place
//   dec_finish (n):          out = sum(share * v) / (sum(share) + eps) in the
//                            query dtype (chunk partials summed in chunk order)
//
// q1 is read in its own dtype and the output stored in it, whatever the
// caches' dtype (the reference loads q1 as fp32 and stores into q1.dtype,
// kernels.py:953, 1029).
//
// HBM bytes per key: K and V rows (2*D*elt) + demand read+write (8) + AFF
// write+read (8).  K and V are streamed once with 16-byte non-temporal loads.
#pragma once

#include "dil_common.hpp"
#include "dil_internal.hpp"
#include "dil_variant.hpp"

namespace dil {

namespace {

// Measured on MI355X at 128K context, B16 H16 d64 bf16 (sweep over 128-1024
// threads, 1-4 rows in flight, 512-8192-key chunks): 1024-thread workgroups
// with two rows in flight per lane over 2048-key chunks stream fastest.
constexpr int kDecThreads = 1024;
constexpr int kDecWaves = kDecThreads / 64;
constexpr int kDecUnroll = 2;          // cached rows in flight per lane

// Keys per workgroup.  At most 2048 (the sweep above), and as many chunks as
// fill whole rounds of the workgroups the GPU holds at once (two 1024-thread
// workgroups per CU, 256 CUs): a partial last round streams at a fraction of
// HBM speed, and a small batch x context would leave CUs idle.  At least 256
// keys.  The rule is computed alike on the host and, for a length held in
// device memory, by the kernels, so both give the same chunks (and the same
// bits) at the same live length.  kDecResident is MI355X's figure (256 CUs x
// 2 workgroups); on a part with another CU count the rule still gives correct
// results, only the last round may then be partly filled.
constexpr int64_t kDecResident = 512;
constexpr int64_t kDecMaxChunk = 2048;
constexpr int64_t kDecMinChunk = 256;

// The chunk count that fills whole rounds: never below the 2048-key count,
// and non-decreasing in `length`.
__host__ __device__ inline int64_t decode_target_chunks(int64_t n, int64_t length) {
  const int64_t base = (length + kDecMaxChunk - 1) / kDecMaxChunk;     // chunks at the largest size
  const int64_t rounds = (n * base + kDecResident - 1) / kDecResident;
  const int64_t target = rounds * kDecResident / n;
  return target < base ? base : target;
}

__host__ __device__ inline int64_t decode_chunk(int64_t n, int64_t length) {
  if (length < 1 || n < 1) return kDecMinChunk;
  const int64_t target = decode_target_chunks(n, length);
  const int64_t chunk = (length + target - 1) / target;
  return chunk < kDecMinChunk ? kDecMinChunk : chunk;
}

// Chunks per slice in the grid and the scratch: exact for a host length; for
// a device-resident live length up to `length`, the largest count of any live
// length.  A live length L <= length has at most target(L) <= target(length)
// chunks (the target does not decrease with the length), and at most one per
// 256 keys.
inline int64_t decode_chunks(int64_t n, int64_t length, bool device_length) {
  if (length < 1) return 1;
  if (!device_length) {
    const int64_t chunk = decode_chunk(n, length);
    return (length + chunk - 1) / chunk;
  }
  const int64_t per_min = (length + kDecMinChunk - 1) / kDecMinChunk;
  const int64_t target = decode_target_chunks(n < 1 ? 1 : n, length);
  return per_min < target ? per_min : target;
}

template <int D>
struct DecLayout {
  static constexpr int kLanesPerRow = D / 8;          // each lane owns 8 consecutive d
  static constexpr int kRowsPerWave = 64 / kLanesPerRow;
  static constexpr int kRowsPerBlock = kRowsPerWave * kDecWaves;
};

// Sum over the kLanesPerRow lanes that share one cached row, with DPP lane
// moves within a 16-lane row (no LDS traffic) and, for 32 lanes, one lane
// shuffle across two rows.  The full sum is guaranteed only in the first lane
// of each row group (lane % LPR == 0), the only lane that consumes it.
template <int LPR>
__device__ __forceinline__ float row_reduce(float x) {
  constexpr int kQuadXor1 = 0xB1;      // quad_perm [1, 0, 3, 2]
  constexpr int kQuadXor2 = 0x4E;      // quad_perm [2, 3, 0, 1]
  constexpr int kRowShl4 = 0x104;      // row_shl:4
  constexpr int kRowShl8 = 0x108;      // row_shl:8
  if constexpr (LPR >= 2)
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kQuadXor1, 0xF, 0xF, true));
  if constexpr (LPR >= 4)
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kQuadXor2, 0xF, 0xF, true));
  if constexpr (LPR >= 8)
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kRowShl4, 0xF, 0xF, true));
  if constexpr (LPR >= 16)
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kRowShl8, 0xF, 0xF, true));
  if constexpr (LPR >= 32) x += __shfl_down(x, 16, 64);   // across the two 16-lane DPP rows (head_dim 256)
  return x;
}

// 8 consecutive cached elements of storage dtype DT as fp32, read with a
// non-temporal hint (the cache is streamed once per step).
template <int DT>
__device__ __forceinline__ void load8_stream(const void* base, int64_t idx, float (&o)[8]) {
  if constexpr (DT == DT_F32) {
    const floatx4* p = reinterpret_cast<const floatx4*>(static_cast<const float*>(base) + idx);
    const floatx4 a = __builtin_nontemporal_load(p), b = __builtin_nontemporal_load(p + 1);
    o[0] = a[0]; o[1] = a[1]; o[2] = a[2]; o[3] = a[3];
    o[4] = b[0]; o[5] = b[1]; o[6] = b[2]; o[7] = b[3];
  } else {
    const u16x8 r = __builtin_nontemporal_load(
        reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(base) + idx));
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = (DT == DT_BF16) ? bf16_bits_to_f32(r[e]) : f16_bits_to_f32(r[e]);
  }
}

// The live length: `length`, or the device-resident value clamped to
// [0, length] (the scratch and the grid are sized for `length`).
__device__ __forceinline__ int64_t live_length(const int64_t* dlen, int64_t length) {
  return dlen == nullptr ? length : max(int64_t{0}, min(*dlen, length));
}
__device__ __forceinline__ int live_chunks(int64_t live, int64_t chunk) {
  return static_cast<int>((live + chunk - 1) / chunk);
}

// Chunk statistics: softmax bids (max, sum 2^(a - max)) in log2 units; ratio
// bids (0 or the minimum of a for minshift, sum of the numerators) in natural
// units; none for the elementwise bids.
template <int D, int DT, int BID = BID_SOFTMAX>
__global__ __launch_bounds__(kDecThreads) void dec_stats(
    const void* __restrict__ q1, int qdt, int64_t q_sn, const void* __restrict__ kc, int64_t kv_sn,
    float* __restrict__ aff, float2* __restrict__ part, int64_t length, int64_t chunk, int nchunk,
    float qscale, int64_t slice0, int64_t nslices, const int64_t* __restrict__ dlen) {
  using L = DecLayout<D>;
  const int64_t slice = slice0 + blockIdx.y;
  const int c = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % L::kLanesPerRow, rw = lane / L::kLanesPerRow;
  const int64_t live = live_length(dlen, length);
  if (dlen != nullptr) chunk = decode_chunk(nslices, live);
  if (c >= live_chunks(live, chunk)) return;             // past the live length: no statistics
  const int64_t j0 = c * chunk;
  const int64_t j1 = min(j0 + chunk, live);

  float q[8];
  load8_f32(q1, slice * q_sn + sub * 8, qdt, q);        // q1 in its own dtype, as fp32
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] *= qscale;

  const int64_t kbase = slice * kv_sn + sub * 8;
  float* arow = aff + slice * length;
  float m = BID == BID_MINSHIFT ? INFINITY : -INFINITY, s = 0.f;
  constexpr int U = kDecUnroll;
  for (int64_t jb = j0 + wave * L::kRowsPerWave + rw; jb < j1; jb += (int64_t)U * L::kRowsPerBlock) {
    float kv[U][8];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + (int64_t)u * L::kRowsPerBlock;
      ok[u] = j < j1;
      if (ok[u]) load8_stream<DT>(kc, kbase + j * D, kv[u]);
    }
    float a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = fmaf(q[e], ok[u] ? kv[u][e] : 0.f, dot);
      a[u] = row_reduce<L::kLanesPerRow>(dot);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + (int64_t)u * L::kRowsPerBlock;
      if (ok[u]) {
        if (sub == 0) arow[j] = a[u];
        tmax = fmaxf(tmax, a[u]);
        if constexpr (bid_ratio<BID>()) {
          if constexpr (BID == BID_MINSHIFT) m = fminf(m, a[u]);
          s += bid_f<BID>(a[u]);
        }
      }
    }
    if (BID == BID_SOFTMAX && tmax > -INFINITY) {
      const float mn = fmaxf(m, tmax);
      float add = 0.f;
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (ok[u]) add += fast_exp2(a[u] - mn);
      s = s * fast_exp2(m - mn) + add;
      m = mn;
    }
  }
  // Lanes of one row hold identical (m, s); count each row once.
  if constexpr (BID != BID_SOFTMAX) {
    if (sub != 0) {                          // only lane sub == 0 holds the full dot products
      s = 0.f;
      m = INFINITY;
    }
    const float wmn = -wave_max(-m);
    const float wsum = wave_sum(s);
    __shared__ float vm[kDecWaves], vs[kDecWaves];
    if (lane == 0) { vm[wave] = wmn; vs[wave] = wsum; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bm = INFINITY, bs = 0.f;
      for (int w = 0; w < kDecWaves; ++w) {
        bm = fminf(bm, vm[w]);
        bs += vs[w];
      }
      part[slice * nchunk + c] = make_float2(bm, bs);
    }
    return;
  }
  if (sub != 0) { m = -INFINITY; s = 0.f; }
  const float wm = wave_max(m);
  float ws = wave_sum(m == -INFINITY ? 0.f : s * fast_exp2(m - wm));
  __shared__ float sm[kDecWaves], ss[kDecWaves];
  if (lane == 0) { sm[wave] = wm; ss[wave] = ws; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bm = -INFINITY;
    for (int w = 0; w < kDecWaves; ++w) bm = fmaxf(bm, sm[w]);
    float bs = 0.f;
    for (int w = 0; w < kDecWaves; ++w)
      if (sm[w] > -INFINITY) bs += ss[w] * fast_exp2(sm[w] - bm);
    part[slice * nchunk + c] = make_float2(bm, bs);
  }
}

template <int D, int DT, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
__global__ __launch_bounds__(kDecThreads) void dec_apply(
    const void* __restrict__ vc, int64_t kv_sn, float* __restrict__ committed, int64_t c_sn,
    const float* __restrict__ aff, const float2* __restrict__ part, float* __restrict__ part_out,
    int64_t length, int64_t chunk, int nchunk, float shift, int64_t slice0, int64_t nslices,
    const int64_t* __restrict__ dlen) {
  using L = DecLayout<D>;
  const int64_t slice = slice0 + blockIdx.y;
  const int c = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % L::kLanesPerRow, rw = lane / L::kLanesPerRow;
  // the scratch strides keep `length` and `nchunk` (the maxima); the walk
  // covers the live length only
  const int64_t live = live_length(dlen, length);
  if (dlen != nullptr) chunk = decode_chunk(nslices, live);
  const int nlive = live_chunks(live, chunk);
  if (c >= nlive) return;

  // Combine the chunk statistics of this slice (every wave redundantly).
  float m = -INFINITY, s = 0.f;
  for (int i = lane; i < nlive; i += 64) {
    const float2 ps = part[slice * nchunk + i];
    const float mn = fmaxf(m, ps.x);
    if (mn > -INFINITY) {
      s = s * fast_exp2(m - mn) + ps.y * fast_exp2(ps.x - mn);
      m = mn;
    }
  }
  const float gm = wave_max(m);
  const float gs = wave_sum(m == -INFINITY ? 0.f : s * fast_exp2(m - gm));
  float lse = gm + __log2f(gs);
  // row parameters of the other bids (natural-unit affinities in AFF)
  float r0 = 0.f, r1 = 0.f;
  const float lshift = __log2f(shift);
  if constexpr (BID != BID_SOFTMAX) {
    float mn = INFINITY, sm = 0.f;
    for (int i = lane; i < nlive; i += 64) {
      const float2 ps = part[slice * nchunk + i];
      mn = fminf(mn, ps.x);
      sm += ps.y;
    }
    mn = -wave_max(-mn);
    sm = wave_sum(sm);
    const float rden = BID == BID_MINSHIFT ? fmaxf(sm - static_cast<float>(live) * mn, 0.f)
                                           : (BID == BID_EXPSHIFT ? shift : sm);
    bid_row_params<BID>(BID == BID_MINSHIFT ? mn : 0.f, rden, static_cast<float>(live), true, r0, r1);
  }

  const int64_t j0 = c * chunk;
  const int64_t j1 = min(j0 + chunk, live);
  const float* arow = aff + slice * length;
  float* crow = committed + slice * c_sn;
  const int64_t vbase = slice * kv_sn + sub * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float ssum = 0.f;
  constexpr int U = kDecUnroll;
  for (int64_t jb = j0 + wave * L::kRowsPerWave + rw; jb < j1; jb += (int64_t)U * L::kRowsPerBlock) {
    float vv[U][8], a[U], cm[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = jb + (int64_t)u * L::kRowsPerBlock;
      ok[u] = j < j1;
      if (ok[u]) {
        load8_stream<DT>(vc, vbase + j * D, vv[u]);
        a[u] = arow[j];
        cm[u] = crow[j];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      const int64_t j = jb + (int64_t)u * L::kRowsPerBlock;
      float p;
      if constexpr (BID == BID_SOFTMAX) p = fast_exp2(a[u] - lse);
      else p = bid_p<BID>(a[u], kLog2e, 1.f, r0, r1, lshift);
      float sh;
      if constexpr (SHARE == SHARE_INCL) sh = p * fast_rcp(cm[u] + p + kEps);
      else if constexpr (SHARE == SHARE_EXCL) sh = p * fast_rcp(cm[u] + kEps);
      else sh = p;
      if (sub == 0) crow[j] = cm[u] + p;
      ssum += sh;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(sh, vv[u][e], acc[e]);
    }
  }
  // Reduce over lanes holding the same d-slice, then over waves.
#pragma unroll
  for (int o = L::kLanesPerRow; o < 64; o <<= 1) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
    ssum += __shfl_xor(ssum, o, 64);
  }
  __shared__ float red[kDecWaves][D + 1];
  if (rw == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) red[wave][sub * 8 + e] = acc[e];
    if (sub == 0) red[wave][D] = ssum;
  }
  __syncthreads();
  for (int i = threadIdx.x; i <= D; i += kDecThreads) {
    float t = 0.f;
    for (int w = 0; w < kDecWaves; ++w) t += red[w][i];
    part_out[(slice * nchunk + c) * (D + 1) + i] = t;
  }
}

// One workgroup (more threads than D) per slice: thread d < D sums column d
// of the chunk partials, thread D the share totals, four chunks at a time.
template <int D>
constexpr int dec_finish_threads() { return D < 256 ? 256 : D + 64; }
template <int D>
__global__ __launch_bounds__(dec_finish_threads<D>()) void dec_finish(const float* __restrict__ part_out, int nchunk,
                                                  void* __restrict__ out, int64_t o_sn, int dt,
                                                  int64_t length, int64_t chunk,
                                                  const int64_t* __restrict__ dlen) {
  const int64_t slice = blockIdx.x;
  const float* base = part_out + slice * nchunk * (D + 1);      // slice stride: the maximum
  const int64_t live = live_length(dlen, length);
  if (dlen != nullptr) chunk = decode_chunk(gridDim.x, live);   // one workgroup per slice
  nchunk = live_chunks(live, chunk);
  __shared__ float tot_s;
  if (threadIdx.x == D) {
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int c = 0;
    for (; c + 4 <= nchunk; c += 4) {
      s0 += base[(c + 0) * (D + 1) + D];
      s1 += base[(c + 1) * (D + 1) + D];
      s2 += base[(c + 2) * (D + 1) + D];
      s3 += base[(c + 3) * (D + 1) + D];
    }
    for (; c < nchunk; ++c) s0 += base[c * (D + 1) + D];
    tot_s = (s0 + s1) + (s2 + s3);
  }
  float t0 = 0.f, t1 = 0.f, t2 = 0.f, t3 = 0.f;
  const int d = threadIdx.x;
  if (d < D) {
    int c = 0;
    for (; c + 4 <= nchunk; c += 4) {
      t0 += base[(c + 0) * (D + 1) + d];
      t1 += base[(c + 1) * (D + 1) + d];
      t2 += base[(c + 2) * (D + 1) + d];
      t3 += base[(c + 3) * (D + 1) + d];
    }
    for (; c < nchunk; ++c) t0 += base[c * (D + 1) + d];
  }
  __syncthreads();
  if (d < D) store_as(out, slice * o_sn + d, dt, ((t0 + t1) + (t2 + t3)) / (tot_s + kEps));
}


template <int D, int DT, int BID = BID_SOFTMAX, int SHARE = SHARE_INCL>
int launch_decode(const DecodeArgs& a) {
  // with a device-resident length the kernels choose the chunk from the live
  // length; the grid and scratch cover every live length up to a.length
  const int64_t chunk = decode_chunk(a.n, a.length);
  const int nchunk = static_cast<int>(decode_chunks(a.n, a.length, a.dlen != nullptr));
  char* ws = static_cast<char*>(a.workspace);
  float* aff = reinterpret_cast<float*>(ws);
  size_t off = align_up(sizeof(float) * a.n * a.length);
  float2* part = reinterpret_cast<float2*>(ws + off);
  off += align_up(sizeof(float2) * a.n * nchunk);
  float* part_out = reinterpret_cast<float*>(ws + off);
  // softmax bids keep log2-unit affinities, the others natural units
  const float qscale = (BID == BID_SOFTMAX ? kLog2e : 1.f) / sqrtf(static_cast<float>(D));
  hipStream_t st = static_cast<hipStream_t>(a.stream);
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    DIL_TIMED("dec_stats", st,
              (dec_stats<D, DT, BID><<<dim3(nchunk, ns), kDecThreads, 0, st>>>(
                  a.q1, a.q_dtype, a.q_sn, a.k_cache, a.kv_sn, aff, part, a.length, chunk, nchunk,
                  qscale, s0, a.n, a.dlen)));
  });
  slice_batches(a.n, [&](int64_t s0, unsigned ns) {
    DIL_TIMED("dec_apply", st,
              (dec_apply<D, DT, BID, SHARE><<<dim3(nchunk, ns), kDecThreads, 0, st>>>(
                  a.v_cache, a.kv_sn, a.committed, a.c_sn, aff, part, part_out, a.length, chunk, nchunk,
                  a.var.shift, s0, a.n, a.dlen)));
  });
  DIL_TIMED("dec_finish", st,
            dec_finish<D><<<dim3(static_cast<unsigned>(a.n)), dec_finish_threads<D>(), 0, st>>>(part_out, nchunk, a.out,
                                                                             a.o_sn, a.q_dtype, a.length,
                                                                             chunk, a.dlen));
  return static_cast<int>(hipGetLastError());
}

}  // namespace
}  // namespace dil
