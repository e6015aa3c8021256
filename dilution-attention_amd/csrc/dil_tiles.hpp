// LDS tile staging, operand fragments and in-register column scans shared by
// the forward and backward kernels (see the layout conventions in
// dil_common.hpp).
#pragma once

#include "dil_common.hpp"

namespace dil {

constexpr int kThreads = 256;   // 4 waves
constexpr int kTileK = 32;      // keys per tile
constexpr int kTileQ = 32;      // query rows per wave

inline int64_t pad64(int64_t x) { return (x + 63) / 64 * 64; }

// Number of 32-wide accumulator tiles along the head dimension (head_dim 16
// uses one tile whose columns >= 16 are padding).
template <int D> constexpr int kDTiles = (D + 31) / 32;

// ---------------------------------------------------------------------------
// operand preparation

// Transposed operand copies are stored tile-major: per slice, for each block
// of 32 rows a contiguous (D, 32) tile, so that one 32-row tile of the
// transpose is a single contiguous 32 * D element read.  Element (row t,
// column d) of a slice sits at (t / 32 * D + d) * 32 + t % 32.
__host__ __device__ inline int64_t tmajor_index(int64_t t, int d, int D) {
  return ((t >> 5) * D + d) * 32 + (t & 31);
}

// Store 8 fp32 values as 8 consecutive CT elements (one 16-byte store for
// bf16, rounded to nearest even; two for fp32 and for a split group, hi then
// lo).  dst is 16-byte aligned (a group start for split).
template <typename CT>
__device__ __forceinline__ void store8(CT* dst, const float (&v)[8]) {
  if constexpr (std::is_same_v<CT, split32>) {
    const SplitFrag f = Mma<split32>::pack(v);
    reinterpret_cast<bf16x8*>(dst)[0] = f.hi;
    reinterpret_cast<bf16x8*>(dst)[1] = f.lo;
  } else if constexpr (sizeof(CT) == 2) {
    *reinterpret_cast<bf16x8*>(dst) = Mma<__bf16>::pack(v);
  } else {
    const floatx4 a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
    reinterpret_cast<floatx4*>(dst)[0] = a;
    reinterpret_cast<floatx4*>(dst)[1] = b;
  }
}

// Load 8 consecutive CT elements (the layout store8 writes) as fp32.
template <typename CT>
__device__ __forceinline__ void load8(const CT* src, float (&v)[8]) {
  if constexpr (std::is_same_v<CT, split32>) {
    const bf16x8* q = reinterpret_cast<const bf16x8*>(src);
    const bf16x8 hi = q[0], lo = q[1];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = static_cast<float>(hi[k]) + static_cast<float>(lo[k]);
  } else if constexpr (sizeof(CT) == 2) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(src);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = static_cast<float>(x[k]);
  } else {
    const floatx4* p = reinterpret_cast<const floatx4*>(src);
    const floatx4 a = p[0], b = p[1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = a[k];
      v[4 + k] = b[k];
    }
  }
}

// One operand preparation: rows of `src` (slice stride src_sn) in the compute
// type, optionally scaled per row by rscale[(slice, row)] (in fp32, before the
// rounding): a row-major copy into dst (slice stride dst_sn) and/or a
// tile-major transposed copy into dst_t.  Null outputs are skipped.
struct PrepJob {
  const void* src;
  int64_t src_sn;
  void* dst;
  int64_t dst_sn;
  void* dst_t;
  const float* rscale;
};

// Up to three preparations of one storage dtype dt and one length, run by one
// launch: blockIdx.z picks the job.
struct PrepJobs {
  PrepJob job[3];
};

// Grid: (row tiles of 64, slices from slice0, jobs).  The transposed copy has
// rows_pad rows (a multiple of 64, zero past `rows`) and slice stride t_sn.
// Every thread stores 16-byte runs: 8 columns of a row in the row-major copy,
// 8 rows of a column in the transposed one (contiguous there, and consecutive
// threads continue the run through the 32 x D block of a 32-row tile).
template <typename CT, int D>
__global__ __launch_bounds__(kThreads) void prep_kernel(PrepJobs jobs, int dt, int64_t rows, int64_t t_sn,
                                                        int64_t rows_pad, int64_t slice0) {
  const PrepJob& job = jobs.job[blockIdx.z];
  const void* __restrict__ src = job.src;
  const int64_t src_sn = job.src_sn, dst_sn = job.dst_sn;
  CT* __restrict__ dst = static_cast<CT*>(job.dst);
  CT* __restrict__ dst_t = static_cast<CT*>(job.dst_t);
  const float* __restrict__ rscale = job.rscale;
  __shared__ float tile[64][D + 1];
  const int64_t slice = slice0 + blockIdx.y;
  const int64_t r0 = static_cast<int64_t>(blockIdx.x) * 64;
  constexpr int kVecPerRow = D / 8;
  for (int idx = threadIdx.x; idx < 64 * kVecPerRow; idx += kThreads) {
    const int r = idx / kVecPerRow, c8 = (idx % kVecPerRow) * 8;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (r0 + r < rows) {
      load8_f32(src, slice * src_sn + (r0 + r) * D + c8, dt, v);
      if (rscale != nullptr) {
        const float f = rscale[slice * rows + r0 + r];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] *= f;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[r][c8 + e] = v[e];
  }
  __syncthreads();
  if (dst != nullptr) {
    for (int idx = threadIdx.x; idx < 64 * kVecPerRow; idx += kThreads) {
      const int r = idx / kVecPerRow, c8 = (idx % kVecPerRow) * 8;
      if (r0 + r < rows) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tile[r][c8 + e];
        store8<CT>(dst + slice * dst_sn + (r0 + r) * D + c8, v);
      }
    }
  }
  if (dst_t != nullptr) {
    // item idx: 32-row half b, column c, rows r8 .. r8 + 7 of that half
    for (int idx = threadIdx.x; idx < 8 * D; idx += kThreads) {
      const int b = idx / (4 * D), c = (idx % (4 * D)) >> 2, r8 = 32 * b + (idx & 3) * 8;
      if (r0 + r8 < rows_pad) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tile[r8 + e][c];
        store8<CT>(dst_t + slice * t_sn + tmajor_index(r0 + r8, c, D), v);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Key groups of the key-parallel passes that form a row-side product (the
// backward's dq, the forward's share V): 8 waves of 32 keys = 256 keys per
// workgroup.  A group's per-(group, 32-row tile) partials are stored
// compactly: key group g meets query tiles [8 g, nq), and tile (g, qt) sits
// at keyq_tile_base(g, nq) + qt - 8 g.

constexpr int kKqWaves = 8;
constexpr int kKqThreads = 64 * kKqWaves;
constexpr int kKqKeys = kKqWaves * kTileK;        // 256 keys per workgroup
constexpr int kKqTilesPerGroup = kKqKeys / kTileQ;  // query tiles spanned by a key group
// bf16 per staged row: the 16-byte pad leaves the 8-byte stage writes and the
// product's 16-byte reads 2-way bank-conflicted (512-byte rows would be
// 16-way); a fully conflict-free layout measured no faster
constexpr int kPdStride = kKqKeys + 8;

// Layout of one partial tile (head_dim 64 x 32 rows) of the key-group
// passes: eight 16 x 16 blocks, block (d / 16, row / 16) at 256 (2 (d / 16) +
// row / 16), each [16 head dims][16 rows].  The wave that forms a block with
// one 16x16x32 MFMA chain stores it as 512 contiguous bytes (lane l: head dim
// l & 15, rows 4 (l >> 4) + [0, 4)), whole cache lines; element e of the tile
// belongs to head dim part_dim(e) and row part_row(e).
__host__ __device__ constexpr int part_block_off(int dq4, int rh, int lane) {
  return 256 * (2 * dq4 + rh) + 16 * (lane & 15) + 4 * (lane >> 4);
}
__host__ __device__ constexpr int part_dim(int e) { return 16 * (e >> 9) + ((e >> 4) & 15); }
__host__ __device__ constexpr int part_row(int e) { return 16 * ((e >> 8) & 1) + (e & 15); }

// The same compact indexing for key groups of KW waves (KW * 32 keys): group
// g meets query tiles [KW g, nq), and tile (g, qt) sits at tile_base(g, nq) +
// qt - KW g.
template <int KW>
struct KeyGroups {
  static constexpr int kWaves = KW;
  static constexpr int kThreads = 64 * KW;
  static constexpr int kKeys = KW * kTileK;
  static constexpr int kTilesPerGroup = kKeys / kTileQ;
  // bf16 per staged [row][key] row: a row stride of 8 banks (mod 128) puts
  // the 16 rows x 2 chunks of a 32-lane 16-byte product read, and the 16 rows
  // of an 8-byte stage write, on distinct banks
  static constexpr int kStride = kKeys + 16;
  __host__ __device__ static int64_t tile_base(int64_t g, int64_t nq) {
    return g * nq - static_cast<int64_t>(kTilesPerGroup) * g * (g - 1) / 2;
  }
  __host__ __device__ static int64_t groups(int64_t T) { return (T + kKeys - 1) / kKeys; }
  __host__ __device__ static int64_t tiles(int64_t T) {
    const int64_t nq = (T + kTileQ - 1) / kTileQ;
    return tile_base(groups(T), nq);
  }
};

// Key groups of KW waves over a chunk of rows [q0, q0 + C) against keys
// [0, q0 + C), q0 a multiple of the group's keys: the a = q0 / (32 KW) groups
// wholly before the chunk meet every one of its nq row tiles, group g >= a
// first meets chunk row tile KW (g - a).  Partial tile (g, rt) sits at
// base(g) + rt - first(g); a chunk at row 0 has the indexing of KeyGroups.
template <int KW>
struct ChunkGroups {
  int64_t nq;   // row tiles of the chunk
  int64_t a;    // key groups wholly before the chunk
  __host__ __device__ int64_t first(int64_t g) const { return g > a ? KW * (g - a) : 0; }
  __host__ __device__ int64_t base(int64_t g) const {
    return g <= a ? g * nq : a * nq + KeyGroups<KW>::tile_base(g - a, nq);
  }
};

__host__ __device__ inline int64_t keyq_tile_base(int64_t g, int64_t nq) {
  return KeyGroups<kKqWaves>::tile_base(g, nq);
}
__host__ __device__ inline int64_t keyq_groups(int64_t T) { return KeyGroups<kKqWaves>::groups(T); }
__host__ __device__ inline int64_t keyq_tiles(int64_t T) { return KeyGroups<kKqWaves>::tiles(T); }

// 16 consecutive floats of LDS into registers (four 16-byte reads).
__device__ __forceinline__ void lds_read16(const float* src, float (&v)[16]) {
  const floatx4* p = reinterpret_cast<const floatx4*>(src);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const floatx4 x = p[u];
    v[4 * u] = x[0];
    v[4 * u + 1] = x[1];
    v[4 * u + 2] = x[2];
    v[4 * u + 3] = x[3];
  }
}

// ---------------------------------------------------------------------------
// LDS staging of 32-row tiles

template <typename CT, int D>
struct Tiles {
  static constexpr int kRowPad = 16 / sizeof(CT);          // 16 B per row breaks bank aliasing
  static constexpr int kKStride = D + kRowPad;              // K tile: [32][D + pad]
  static constexpr int kTStride = kTileK + kRowPad;         // transposed tile: [D][32 + pad]
  static constexpr int kChunk = 16 / sizeof(CT);            // elements per 16-byte copy
  static constexpr int kKChunks = kTileK * D / kChunk;      // 16-byte chunks per K tile
  static constexpr int kTChunks = D * kTileK / kChunk;
};

template <typename CT> struct Vec16 { typedef floatx4 type; };
template <> struct Vec16<__bf16> { typedef bf16x8 type; };

// The tile loaders below split a copy global -> LDS into load() at the start
// of a step and store() at its end.  In the buffer and clamp forms every
// thread issues its loads unconditionally: with no branch around a load the
// compiler waits for the loads only where store() consumes them, so they
// overlap the whole step.  The buffer form loads through a resource whose
// base is the wave-uniform tile address and whose size ends at the slice's
// last row, with a 32-bit per-lane offset: chunks past the end read as zeros
// without touching memory, and no 64-bit per-lane address is kept or advanced
// across the loop.  The clamp form clamps its addresses into the slice and
// zeroes the rows past the end in store().  The skip form loads only the rows
// inside the slice, each under its own condition.

// Raw buffer resource (gfx9: stride 0, word 3 = 0x00020000) over `bytes`
// bytes at `base`.  Both must be the same in every lane of the wave (every
// caller passes a tile or row address shared by the workgroup or the wave);
// readfirstlane states that to the compiler, which then builds the resource
// in scalar registers instead of looping over the distinct per-lane values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
  const int64_t n = bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes);
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(a >> 32));
  void* ub = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, __builtin_amdgcn_readfirstlane(static_cast<int>(n)), 0x00020000);
}
// 16 bytes at byte offset voff (per lane) + soff (uniform); zeros past the end.
template <typename V>
__device__ __forceinline__ V buffer_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
__device__ __forceinline__ float buffer_load_f32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
// Loads of a split reduction's partials, which are read exactly once: the
// non-temporal hint streams them past the caches instead of evicting reused
// data (measured 11% faster on the partial reductions).
__device__ __forceinline__ bf16x8 load_once(const __bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}
__device__ __forceinline__ float load_once(const float* p) { return __builtin_nontemporal_load(p); }

// The main loop of a double-buffered kernel: iter(i, buf) for i in [begin,
// end), with LDS buffer buf = (i - begin) & 1.  UNROLL unrolls it by two so
// that buf is a constant in each copy and the buffer offsets fold into the
// LDS instructions (about 10 VALU per step less); kernels whose registers are
// at their limit keep the plain loop.
template <bool UNROLL, typename I, typename F>
__device__ __forceinline__ void double_buffered(I begin, I end, F&& iter) {
  if constexpr (UNROLL) {
    I i = begin;
    for (; i + 1 < end; i += 2) {
      iter(i, 0);
      iter(i + 1, 1);
    }
    if (i < end) iter(i, 0);
  } else {
    int buf = 0;
    for (I i = begin; i < end; ++i, buf ^= 1) iter(i, buf);
  }
}

// Slot of row r when a 32-row tile is stored in the query-split order of
// qsig() (slot m holds row qsig(m)): the inverse of qsig.
__device__ __forceinline__ int qs_slot(int r) { return (((r >> 2) & 3) << 3) | (((r >> 4) & 1) << 2) | (r & 3); }

// How a tile loader reads global memory (see above): through a buffer
// resource, from addresses clamped into the slice, or (skip) only the rows
// inside the slice, each load under its own condition.  Which one is fastest
// depends on the kernel; each kernel uses the one measured best for it.
enum LoadMode { kLoadBuffer = 0, kLoadClamp = 1, kLoadSkip = 2 };

// Copy one K tile (rows [key0, key0+32) of a row-major (rows, D) slice with
// nkeys >= 1 rows) into registers: each thread owns kKChunks / kThreads
// 16-byte chunks; rows past nkeys end up as zeros.  QS stores the rows in
// query-split order (row r at slot qs_slot(r)): lanes that read rows qsig(l)
// then read consecutive slots, which keeps their 16-byte LDS reads free of
// bank conflicts (rows r and r + 16 of the natural order share banks).
template <typename CT, int D, bool QS = false, int MODE = kLoadBuffer>
struct KTileLoader {
  using T = Tiles<CT, D>;
  using V = typename Vec16<CT>::type;
  static constexpr int kPer = (T::kKChunks + kThreads - 1) / kThreads;
  static constexpr int kPerRow = D / T::kChunk;
  V r[kPer];
  int nrows;                                        // rows inside the slice (clamp form)
  __device__ void load(const CT* base, int64_t key0, int64_t nkeys) {
    if constexpr (MODE == kLoadBuffer) {
      const int64_t rows = min(max(nkeys - key0, int64_t{0}), int64_t{kTileK});
      const auto rs = make_rsrc(base + key0 * D, rows * D * static_cast<int64_t>(sizeof(CT)));
#pragma unroll
      for (int u = 0; u < kPer; ++u)   // chunks idx >= kKChunks lie past the tile: zeros, never stored
        r[u] = buffer_load16<V>(rs, static_cast<uint32_t>((threadIdx.x + u * kThreads) * 16), 0);
    } else {
      // slices hold fewer than 2^31 rows
      const int k0 = static_cast<int>(key0), last = static_cast<int>(nkeys) - 1;
      nrows = min(max(last + 1 - k0, 0), kTileK);
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        if constexpr (MODE == kLoadClamp) {
          const int idx = min(static_cast<int>(threadIdx.x) + u * kThreads, T::kKChunks - 1);
          const int row = min(k0 + idx / kPerRow, last);
          r[u] = *reinterpret_cast<const V*>(base + static_cast<int64_t>(row) * D + (idx % kPerRow) * T::kChunk);
        } else {
          const int idx = threadIdx.x + u * kThreads;
          const int row = idx / kPerRow;
          r[u] = V{};
          if (idx < T::kKChunks && row < nrows)
            r[u] = *reinterpret_cast<const V*>(base + (key0 + row) * D + (idx % kPerRow) * T::kChunk);
        }
      }
    }
  }
  __device__ void store(CT* lds) const {
    const bool full = MODE != kLoadClamp || nrows == kTileK;   // workgroup-uniform
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      const int row = idx / kPerRow, c = (idx % kPerRow) * T::kChunk;
      const int slot = QS ? qs_slot(row) : row;
      if (idx < T::kKChunks)
        *reinterpret_cast<V*>(lds + slot * T::kKStride + c) = (full || row < nrows) ? r[u] : V{};
    }
  }
};

// Copy one transposed tile (rows d in [0, D), columns [key0, key0 + 32), key0
// a multiple of 32) of a tile-major slice into registers: 32 * D contiguous
// elements.
// DSTRIDE: the head dims of the tile-major copy, when the loader takes only
// D of them (base then points at the first taken row of the first tile).
template <typename CT, int D, int MODE = kLoadBuffer, int DSTRIDE = D>
struct TTileLoader {
  using T = Tiles<CT, D>;
  using V = typename Vec16<CT>::type;
  static constexpr int kPer = (T::kTChunks + kThreads - 1) / kThreads;
  static constexpr int kPerRow = kTileK / T::kChunk;
  V r[kPer];
  __device__ void load(const CT* base, int64_t key0) {
    const CT* tile = base + key0 * DSTRIDE;         // (key0 / 32) * DSTRIDE * 32: the tile's first element
    if constexpr (MODE == kLoadBuffer) {
      const auto rs = make_rsrc(tile, kTileK * D * static_cast<int64_t>(sizeof(CT)));
#pragma unroll
      for (int u = 0; u < kPer; ++u)   // chunks idx >= kTChunks lie past the tile: zeros, never stored
        r[u] = buffer_load16<V>(rs, static_cast<uint32_t>((threadIdx.x + u * kThreads) * 16), 0);
    } else {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int idx = min(static_cast<int>(threadIdx.x) + u * kThreads, T::kTChunks - 1);
        r[u] = *reinterpret_cast<const V*>(tile + idx * T::kChunk);
      }
    }
  }
  __device__ void store(CT* lds) const {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int idx = threadIdx.x + u * kThreads;
      const int d = idx / kPerRow, c = (idx % kPerRow) * T::kChunk;
      if (idx < T::kTChunks) *reinterpret_cast<V*>(lds + d * T::kTStride + c) = r[u];
    }
  }
};

// Row fragment of a 32-row tile held in LDS ([32][kKStride]); lane reads row `row`.
template <typename CT, int D>
__device__ __forceinline__ void lds_row_frag(RowFrag<CT, D>& rf, const CT* lds, int row, int h) {
  load_row_frag<CT, D>(rf, lds + row * Tiles<CT, D>::kKStride + h * (D / 2));
}

// Operand fragment over 32 keys from a transposed LDS tile ([D][kTStride]):
// lane (row r of the D dimension, half h) supplies, for instruction s, the
// keys that the permuted accumulator layout assigns to k slots of half h:
// bf16: keys 16 s + 8 h + [0, 8); fp32: key perm_row(s, h).
template <typename CT, int D>
__device__ __forceinline__ typename Mma<CT>::frag lds_t_frag(const CT* lds, int r, int h, int s) {
  if (D < 32 && r >= D) return typename Mma<CT>::frag{};
  const CT* row = lds + r * Tiles<CT, D>::kTStride;
  if constexpr (kWideFrag<CT>) {
    return frag8_at<CT>(row + 16 * s + 8 * h);
  } else {
    return row[perm_row(s, h)];
  }
}

// Operand fragment built from 16 accumulator values of one lane (the
// permuted layout): instruction s takes registers [s*kPerLane, (s+1)*kPerLane).
template <typename CT>
__device__ __forceinline__ typename Mma<CT>::frag acc_frag(const float* v, int s) {
  return Mma<CT>::pack(v + s * Mma<CT>::kPerLane);
}

// Identity operand that transposes a 32x32 accumulator tile held in the
// permuted layout: B[k][n] = 1 where k (the logical row of slot t of
// instruction s in half h) equals n = lane & 31.
template <typename CT>
__device__ __forceinline__ typename Mma<CT>::frag ident_frag(int l32, int h, int s) {
  if constexpr (kWideFrag<CT>) {
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = (16 * s + 8 * h + t == l32) ? 1.f : 0.f;
    return Mma<CT>::pack(v);
  } else {
    return (perm_row(s, h) == l32) ? 1.f : 0.f;
  }
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for
// every outstanding global load and store of the wave (its fence covers global
// memory), which would cut the prefetch of the next tile and put the
// checkpoint stores on the critical path of every step.  The tile loops
// exchange data between waves through LDS only, so they synchronise with this.
__device__ __forceinline__ void sync_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum of 16 values as a depth-4 tree.
__device__ __forceinline__ float sum16(const float (&v)[16]) {
  float a[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) a[k] = v[k] + v[k + 8];
#pragma unroll
  for (int k = 0; k < 4; ++k) a[k] += a[k + 4];
  return (a[0] + a[2]) + (a[1] + a[3]);
}

// 16 per-register values as an accumulator (the initial value of a product).
__device__ __forceinline__ floatx16 as_x16(const float (&v)[16]) {
  floatx16 r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = v[i];
  return r;
}

// ---------------------------------------------------------------------------
// XCD-aware work mapping.
//
// The dispatcher hands workgroups to the 8 XCDs of an MI355X round-robin by
// linear workgroup id, and each XCD has its own L2.  Work item L of a 1-D
// grid of kXcds * per workgroups goes to workgroup b with
// L = (b % kXcds) * per + b / kXcds, so an XCD runs a contiguous range of
// items: consecutive tiles of the same (batch, head) slice, whose K/V (or
// Q/dO) streams then stay in that XCD's L2.

constexpr int kXcds = 8;

inline int64_t xcd_grid(int64_t items) { return kXcds * ((items + kXcds - 1) / kXcds); }

// Whether a call's workgroups go out longest first (xcd_work_item): measured
// faster for calls of up to 2^18 tokens (slices x keys: -3% to -12% on the
// training step at T = 2048 ... 16384), slower beyond (+1.6% on the 2^20
// tokens of a B4 H16 T16384 call), where all of an XCD's slices in flight at
// once miss in its L2 more than the packing gains.  Rows of at most 2048 keys
// go longest first at any slice count: their walks are short, so the tail of
// the longest ones matters more than L2 locality (B32 H12 T1024 fwd+bwd
// 1.07 -> 1.00 ms).
inline bool longest_first_for(int64_t slices, int64_t keys) {
  return slices * keys <= (int64_t{1} << 18) || keys <= 2048;
}

struct WorkItem {
  int64_t slice;
  int idx;       // tile-group index within the slice, in dispatch order
  bool valid;
};

// items = groups * slices; group idx 0 of a slice is its heaviest item
// (`reverse` maps the order 0, 1, ... to groups - 1, ..., 0).  Workgroups
// reach the XCDs round-robin (block b on XCD b % 8), and each XCD takes a
// contiguous share of the slices so that their tiles stay in its L2.  When
// the slices divide evenly over the XCDs, an XCD dispatches its items
// longest first across all of its slices (group 0 of every slice, then group
// 1, ...): dispatched slice by slice instead, the heaviest items of its last
// slices start near the end and run alone, which left ~30% of the slots idle
// with 16 slices of 16 groups per XCD.  Otherwise, or with !longest_first
// (a kernel with little arithmetic per byte, for which more slices in flight
// per XCD cost more in L2 misses than the packing gains), the items are
// split into contiguous ranges, slice by slice.  With `spread` (a kernel whose
// items read little that they share) slices that do not divide evenly go out
// longest first over the whole chip instead: block b takes the rank b / slices
// of slice b % slices, so every XCD gets its share of the long and the short
// items (in contiguous ranges, two slices of 512 groups left the XCD holding
// the longest walks with 7x the work of the one holding the shortest).
__device__ __forceinline__ WorkItem xcd_work_item(int groups, int64_t slices, bool reverse,
                                                 bool longest_first = true, bool spread = false) {
  const int64_t b = blockIdx.x;
  WorkItem w;
  int r;
  if (longest_first && slices % kXcds == 0) {
    const int64_t spx = slices / kXcds, j = b / kXcds;     // slices per XCD, rank on the XCD
    w.valid = j < spx * groups;
    r = static_cast<int>(j / spx);
    w.slice = (b % kXcds) * spx + j % spx;
  } else if (longest_first && spread) {
    w.valid = b < static_cast<int64_t>(groups) * slices;
    r = static_cast<int>(b / slices);
    w.slice = b % slices;
  } else {
    const int64_t total = static_cast<int64_t>(groups) * slices;
    const int64_t per = (total + kXcds - 1) / kXcds;
    const int64_t L = (b % kXcds) * per + b / kXcds;
    w.valid = L < total;
    w.slice = L / groups;
    r = static_cast<int>(L % groups);
  }
  w.idx = reverse ? groups - 1 - r : r;
  return w;
}

// ---------------------------------------------------------------------------
// Query-split tile layout ("QS")
//
// A score tile S = Q K^T whose A operand (Q) is loaded with lane m holding
// query row qsig(m) puts, in accumulator register i of lane half h, the query
// 16 h + i: half 0 holds rows 0..15 and half 1 rows 16..31, each in register
// order.  A column (one key per lane) then scans down its 32 rows as one
// 16-long register chain per half plus one exchange between the halves.
// Contracting over those rows (dv += dO^T A, dk += Q^T (p dp)) uses operand
// k slots 16 h + 8 s + [0, 8) (bf16) or 16 h + s (fp32) of a transposed tile.

__device__ __forceinline__ int qsig(int m) { return 16 * ((m >> 2) & 1) + 4 * (m >> 3) + (m & 3); }

// Values of x in the two lanes of the pair (l & 31, (l & 31) + 32), in every
// lane of the pair: .lo from the lower-half lane, .hi from the upper-half lane.
struct HalfPair {
  float lo, hi;
};
__device__ __forceinline__ HalfPair halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return HalfPair{__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// Operand fragment over 32 QS-ordered rows of a transposed LDS tile
// ([D][kTStride]); lane supplies row r of the D dimension.
template <typename CT, int D>
__device__ __forceinline__ typename Mma<CT>::frag lds_tq_frag(const CT* lds, int r, int h, int s) {
  if (D < 32 && r >= D) return typename Mma<CT>::frag{};
  const CT* row = lds + r * Tiles<CT, D>::kTStride;
  if constexpr (kWideFrag<CT>) {
    return frag8_at<CT>(row + 16 * h + 8 * s);
  } else {
    return row[16 * h + s];
  }
}

// Identity operand that transposes a QS-layout tile: B[k][n] = 1 where the
// query held in k slot k equals n = lane & 31.
template <typename CT>
__device__ __forceinline__ typename Mma<CT>::frag ident_qs(int l32, int h, int s) {
  if constexpr (kWideFrag<CT>) {
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = (16 * h + 8 * s + t == l32) ? 1.f : 0.f;
    return Mma<CT>::pack(v);
  } else {
    return (16 * h + s == l32) ? 1.f : 0.f;
  }
}

// B operand that appends a ones column to a product over 32 k slots: column 0
// of the 32-wide output tile receives the sum of the A operand's row over k.
template <typename CT>
__device__ __forceinline__ typename Mma<CT>::frag ones_col_frag(int l32) {
  if constexpr (kWideFrag<CT>) {
    const float v = l32 == 0 ? 1.f : 0.f;
    const float w[8] = {v, v, v, v, v, v, v, v};
    return Mma<CT>::pack(w);
  } else {
    return l32 == 0 ? 1.f : 0.f;
  }
}

// Inclusive column scan of a QS-layout tile: x[i] becomes base + the sum of
// the column's entries at rows <= 16 h + i.  hf = float(h).  Returns the
// column total (excluding base).
__device__ __forceinline__ float scan_incl_qs(float (&x)[16], float base, float hf) {
#pragma unroll
  for (int t = 1; t < 16; ++t) x[t] += x[t - 1];
  const HalfPair tot = halves(x[15]);
  const float off = fmaf(hf, tot.lo, base);
#pragma unroll
  for (int t = 0; t < 16; ++t) x[t] += off;
  return tot.lo + tot.hi;
}

// Exclusive column scan of a QS-layout tile: x[i] becomes base + the sum of
// the column's entries at rows < 16 h + i (no subtraction, so an entry with no
// earlier mass is exactly `base`).  Returns the column total.
__device__ __forceinline__ float scan_excl_qs(float (&x)[16], float base, float hf) {
  float run = 0.f;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const float cur = x[t];
    x[t] = run;
    run += cur;
  }
  const HalfPair tot = halves(run);
  const float off = fmaf(hf, tot.lo, base);
#pragma unroll
  for (int t = 0; t < 16; ++t) x[t] += off;
  return tot.lo + tot.hi;
}

// Inclusive suffix scan of a QS-layout tile: x[i] becomes base + the sum of
// the column's entries at rows >= 16 h + i.  Returns the column total.
__device__ __forceinline__ float scan_suffix_qs(float (&x)[16], float base, float hf) {
#pragma unroll
  for (int t = 14; t >= 0; --t) x[t] += x[t + 1];
  const HalfPair tot = halves(x[0]);
  const float off = fmaf(1.f - hf, tot.hi, base);
#pragma unroll
  for (int t = 0; t < 16; ++t) x[t] += off;
  return tot.lo + tot.hi;
}

// Column scan over the 32 rows of an accumulator tile in the permuted layout
// (register i of half h = row 16*(i>>3) + 8*h + (i&7)).  On return x[i] holds
// base + sum of the column's entries at rows <= row(i): the inclusive demand
// plus `base`.  Also returns the column total (the same in both halves).
__device__ __forceinline__ float column_scan_inclusive(float (&x)[16], float base, int h) {
  // inclusive prefix within each run of 8
#pragma unroll
  for (int t = 1; t < 8; ++t) x[t] += x[t - 1];
#pragma unroll
  for (int t = 9; t < 16; ++t) x[t] += x[t - 1];
  const float tlo = x[7], thi = x[15];
  const float plo = partner32(tlo), phi = partner32(thi);
  // column order: [h0 lo][h1 lo][h0 hi][h1 hi]
  const float off_lo = h ? plo : 0.f;
  const float off_hi = h ? (plo + tlo + phi) : (tlo + plo);
  const float blo = base + off_lo, bhi = base + off_hi;
#pragma unroll
  for (int t = 0; t < 8; ++t) x[t] += blo;
#pragma unroll
  for (int t = 8; t < 16; ++t) x[t] += bhi;
  return tlo + thi + plo + phi;
}


// Reverse (suffix) scan over the 32 rows of an accumulator tile in the
// permuted layout.  On return x[i] holds base + the sum of the column's
// entries at rows strictly after row(i).  Returns the column total.
__device__ __forceinline__ float column_scan_suffix_exclusive(float (&x)[16], float base, int h) {
  float s = 0.f;
#pragma unroll
  for (int t = 7; t >= 0; --t) {
    const float v = x[t];
    x[t] = s;
    s += v;
  }
  const float tlo = s;
  s = 0.f;
#pragma unroll
  for (int t = 15; t >= 8; --t) {
    const float v = x[t];
    x[t] = s;
    s += v;
  }
  const float thi = s;
  const float plo = partner32(tlo), phi = partner32(thi);
  // column order: [h0 lo][h1 lo][h0 hi][h1 hi]; add what lies after each run
  const float off_lo = base + (h ? (phi + thi) : (plo + thi + phi));
  const float off_hi = base + (h ? 0.f : phi);
#pragma unroll
  for (int t = 0; t < 8; ++t) x[t] += off_lo;
#pragma unroll
  for (int t = 8; t < 16; ++t) x[t] += off_hi;
  return tlo + thi + plo + phi;
}

}  // namespace dil
