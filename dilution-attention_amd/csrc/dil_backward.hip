// Entry points of the backward: the production operator for head_dim 16-128
// in every precision and for 256 with bf16 operands; the ablation variants are
// built in dil_variants.hip (head_dim 16-128) and reached through
// backward_bid<BID>.
#include "dil_backward_impl.hpp"

namespace dil {

namespace {

template <int D>
int dispatch_backward(const BackwardArgs& a) {
  switch (a.prec) {
    case 2: return launch_backward<__bf16, D>(a);
    case 1: return launch_backward<split32, D>(a);
    default: return launch_backward<float, D>(a);
  }
}

}  // namespace

int64_t backward_workspace_bytes(int64_t n, int64_t T, int head_dim, int dtype, int prec) {
  // sized with dout needing conversion (the larger case)
  return static_cast<int64_t>(
      bwd_layout(n, T, head_dim, dtype, prec == 2 ? DT_F32 : DT_BF16, prec).total);
}

int backward(const BackwardArgs& a) {
  if (const int err = check_variant(a.var, a.head_dim)) return err;
  if (a.var.bid != BID_SOFTMAX || a.var.share != SHARE_INCL) {
    switch (a.var.bid) {
      case 0: return backward_bid<0>(a);
      case 1: return backward_bid<1>(a);
      case 2: return backward_bid<2>(a);
      case 3: return backward_bid<3>(a);
      case 4: return backward_bid<4>(a);
      case 5: return backward_bid<5>(a);
      case 6: return backward_bid<6>(a);
      default: return backward_bid<7>(a);
    }
  }
  switch (a.head_dim) {
    case 16: return dispatch_backward<16>(a);
    case 32: return dispatch_backward<32>(a);
    case 64: return dispatch_backward<64>(a);
    case 128: return dispatch_backward<128>(a);
    case 256: return a.prec == 2 ? launch_backward<__bf16, 256>(a) : kErrHeadDim;
    default: return kErrHeadDim;
  }
}

}  // namespace dil
