// Entry points of the cached decode step: the production operator for every
// head_dim (16-256) and dtype; the ablation variants are built in
// dil_variants.hip (head_dim 16-128) and reached through decode_bid<BID>.
#include "dil_decode_impl.hpp"

namespace dil {

// Sized for a device-resident length up to `length` (the larger chunk count),
// so one size serves dil_decode_step and dil_decode_step_dlen.
int64_t decode_workspace_bytes(int64_t n, int64_t length, int head_dim) {
  const int64_t nchunk = decode_chunks(n, length, true);
  return static_cast<int64_t>(align_up(sizeof(float) * n * length) +
                              align_up(sizeof(float2) * n * nchunk) +
                              align_up(sizeof(float) * n * nchunk * (head_dim + 1)));
}

template <int D>
int decode_dtype(const DecodeArgs& a) {
  switch (a.dtype) {
    case DT_F32: return launch_decode<D, DT_F32>(a);
    case DT_BF16: return launch_decode<D, DT_BF16>(a);
    case DT_F16: return launch_decode<D, DT_F16>(a);
    default: return kErrDtype;
  }
}

int decode_step(const DecodeArgs& a) {
  if (const int err = check_variant(a.var, a.head_dim)) return err;
  if (a.var.bid != BID_SOFTMAX || a.var.share != SHARE_INCL) {
    switch (a.var.bid) {
      case 0: return decode_bid<0>(a);
      case 1: return decode_bid<1>(a);
      case 2: return decode_bid<2>(a);
      case 3: return decode_bid<3>(a);
      case 4: return decode_bid<4>(a);
      case 5: return decode_bid<5>(a);
      case 6: return decode_bid<6>(a);
      default: return decode_bid<7>(a);
    }
  }
  switch (a.head_dim) {
    case 16: return decode_dtype<16>(a);
    case 32: return decode_dtype<32>(a);
    case 64: return decode_dtype<64>(a);
    case 128: return decode_dtype<128>(a);
    case 256: return decode_dtype<256>(a);
    default: return kErrHeadDim;
  }
}

}  // namespace dil
