// Entry points of the forward (plain forward and chunked prefill): the
// production operator for head_dim 16-128 in every precision and for 256 with
// bf16 operands; the ablation variants are built in dil_variants.hip (head_dim
// 16, 32, 64 and 128) and reached through forward_bid<BID>.
#include "dil_forward_impl.hpp"

namespace dil {

namespace {

template <int D>
int dispatch_forward(const ForwardArgs& a) {
  switch (a.prec) {
    case 2: return launch_forward<__bf16, D>(a);
    case 1: return launch_forward<split32, D>(a);
    default: return launch_forward<float, D>(a);
  }
}

}  // namespace

int64_t forward_workspace_bytes(int64_t n, int64_t C, int64_t Tk, int head_dim, int dtype, int prec,
                                int want_pk, bool key_pass) {
  return static_cast<int64_t>(fwd_layout(n, C, Tk, head_dim, dtype, prec, want_pk, key_pass).total);
}

bool forward_takes_key_pass(int64_t C, int64_t Tk, int64_t q0, int head_dim, int prec, const Variant& var,
                            bool key_pass) {
  return var.bid == BID_SOFTMAX && var.share == SHARE_INCL && keyout_eligible(C, Tk, q0, head_dim, prec, key_pass);
}

int forward(const ForwardArgs& a) {
  if (const int err = check_variant(a.var, a.head_dim)) return err;
  // no checkpoint array: only the key pass can do without it
  if (a.carry == nullptr && !forward_takes_key_pass(a.C, a.Tk, a.q0, a.head_dim, a.prec, a.var, a.key_pass))
    return kErrShape;
  if (a.var.bid != BID_SOFTMAX || a.var.share != SHARE_INCL) {
    switch (a.var.bid) {
      case 0: return forward_bid<0>(a);
      case 1: return forward_bid<1>(a);
      case 2: return forward_bid<2>(a);
      case 3: return forward_bid<3>(a);
      case 4: return forward_bid<4>(a);
      case 5: return forward_bid<5>(a);
      case 6: return forward_bid<6>(a);
      default: return forward_bid<7>(a);
    }
  }
  switch (a.head_dim) {
    case 16: return dispatch_forward<16>(a);
    case 32: return dispatch_forward<32>(a);
    case 64: return dispatch_forward<64>(a);
    case 128: return dispatch_forward<128>(a);
    case 256: return a.prec == 2 ? launch_forward<__bf16, 256>(a) : kErrHeadDim;
    default: return kErrHeadDim;
  }
}

}  // namespace dil
