// Ablation variants of one bid function, the reference's kernels_bid.py
// operator family (src/dilution/kernels_bid.py): forward, backward and cached
// decode for the three share modes, head_dim 16 / 32 / 64 / 128, bf16 and fp32
// MFMA operands.
// This file is compiled once per bid with -DDIL_VARIANT_BID=<0..7> into its
// own object; the entry points dispatch non-production variants here.
#include <type_traits>

#include "dil_backward_impl.hpp"
#include "dil_decode_impl.hpp"
#include "dil_forward_impl.hpp"

#ifndef DIL_VARIANT_BID
#error "compile with -DDIL_VARIANT_BID=<bid 0..7>"
#endif

namespace dil {

namespace {

constexpr int kB = DIL_VARIANT_BID;

// f<D>() for the call's head_dim (validated by the entry points)
template <typename F>
int with_head_dim(int head_dim, F&& f) {
  switch (head_dim) {
    case 16: return f(std::integral_constant<int, 16>{});
    case 32: return f(std::integral_constant<int, 32>{});
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    default: return kErrHeadDim;
  }
}

template <int SHARE>
int forward_share(const ForwardArgs& a) {
  if constexpr (is_production<kB, SHARE>()) {
    return kErrVariant;                      // the production operator is built in dil_forward.hip
  } else {
    // the ablation variants run "tf32" on fp32 operands
    return with_head_dim(a.head_dim, [&](auto d) {
      constexpr int D = decltype(d)::value;
      return a.prec == 2 ? launch_forward<__bf16, D, kB, SHARE>(a) : launch_forward<float, D, kB, SHARE>(a);
    });
  }
}

template <int SHARE>
int backward_share(const BackwardArgs& a) {
  if constexpr (is_production<kB, SHARE>()) {
    return kErrVariant;
  } else {
    return with_head_dim(a.head_dim, [&](auto d) {
      constexpr int D = decltype(d)::value;
      return a.prec == 2 ? launch_backward<__bf16, D, kB, SHARE>(a) : launch_backward<float, D, kB, SHARE>(a);
    });
  }
}

template <int SHARE>
int decode_share(const DecodeArgs& a) {
  if constexpr (is_production<kB, SHARE>()) {
    return kErrVariant;
  } else {
    return with_head_dim(a.head_dim, [&](auto d) {
      constexpr int D = decltype(d)::value;
      switch (a.dtype) {
        case DT_F32: return launch_decode<D, DT_F32, kB, SHARE>(a);
        case DT_BF16: return launch_decode<D, DT_BF16, kB, SHARE>(a);
        case DT_F16: return launch_decode<D, DT_F16, kB, SHARE>(a);
        default: return kErrDtype;
      }
    });
  }
}

}  // namespace

template <int BID>
int forward_bid(const ForwardArgs& a) {
  static_assert(BID == kB, "one bid per object");
  switch (a.var.share) {
    case SHARE_NONE: return forward_share<SHARE_NONE>(a);
    case SHARE_INCL: return forward_share<SHARE_INCL>(a);
    default: return forward_share<SHARE_EXCL>(a);
  }
}

template <int BID>
int backward_bid(const BackwardArgs& a) {
  static_assert(BID == kB, "one bid per object");
  switch (a.var.share) {
    case SHARE_NONE: return backward_share<SHARE_NONE>(a);
    case SHARE_INCL: return backward_share<SHARE_INCL>(a);
    default: return backward_share<SHARE_EXCL>(a);
  }
}

template <int BID>
int decode_bid(const DecodeArgs& a) {
  static_assert(BID == kB, "one bid per object");
  switch (a.var.share) {
    case SHARE_NONE: return decode_share<SHARE_NONE>(a);
    case SHARE_INCL: return decode_share<SHARE_INCL>(a);
    default: return decode_share<SHARE_EXCL>(a);
  }
}

template int forward_bid<DIL_VARIANT_BID>(const ForwardArgs&);
template int backward_bid<DIL_VARIANT_BID>(const BackwardArgs&);
template int decode_bid<DIL_VARIANT_BID>(const DecodeArgs&);

}  // namespace dil
