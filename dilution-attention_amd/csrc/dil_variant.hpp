// Bid functions and share modes of the operator's ablation variants.
//
// Reference behaviour: src/dilution/kernels_bid.py.  The bid p_ij of query i
// for key j (kernels_bid.py:4-42, bids_from_affinity :94-121, in-kernel
// _p_jac_from_k :184-226), with a = q_i.k_j / sqrt(D) on the causal window:
//
//   BID 0 softmax   p = softmax_j(a)                      jac = p
//   BID 1 relu      p = relu(a) / R                      jac = 1[a > 0] / R
//   BID 2 relu2     p = relu(a)^2 / R                    jac = 2 relu(a) / R
//   BID 3 softplus  p = softplus(a) / R                  jac = sigmoid(a) / R
//   BID 4 minshift  p = (a - min_window a) / R           jac = 1 / R (the min held constant)
//   BID 5 sigmoid   p = sigmoid(a)                       jac = p (1 - p)
//   BID 6 expshift  p = exp(a) / SHIFT                   jac = p
//   BID 7 sigshift  p = 1 / (1 + SHIFT e^-a)             jac = p (1 - p)
//
// R is the row sum of the numerator over the window; a row with R = 0 bids
// uniformly, 1 / (window length), with zero Jacobian.  Bids 0-4 are row
// normalised, so their backward carries the ghat term; 5-7 are elementwise.
// The share step (kernels_bid.py:248-265):
//
//   SHARE 1 (dilution)   share = p / (committed + p + eps)
//   SHARE 2 (exclusive)  share = p / (committed + eps)
//   SHARE 0 (none)       share = p
//
// then share / rowsum(share) @ V in every mode.  The kernels recompute p from
// two per-row parameters (r0, r1) held in LDS next to the tiles:
//
//   log2 bids (0, 6):    p = 2^(a log2(e) - r0), r0 = log2-sum-exp of the row
//                        (log2 SHIFT for expshift); +inf on rows past the end
//   ratio bids (1-4):    p = f(a) r0 - r1 (two rounded operations, never an fma),
//                        r0 = 1 / R (0 for an empty row), r1 = (min a) r0
//                        for minshift, -1 / window on an empty row, else 0;
//                        both 0 on rows past the end.  For minshift f(a) = a,
//                        so the row's minimum gets exactly p = 0 and no key
//                        gets a negative bid (the recomputed products are
//                        bitwise those of the statistics pass).
//   sigmoid bids (5, 7): p = r0 sigmoid(a - log SHIFT), r0 = 1 on a row, 0 past the end
#pragma once

#include "dil_common.hpp"

namespace dil {

enum : int {
  BID_SOFTMAX = 0,
  BID_RELU = 1,
  BID_RELU2 = 2,
  BID_SOFTPLUS = 3,
  BID_MINSHIFT = 4,
  BID_SIGMOID = 5,
  BID_EXPSHIFT = 6,
  BID_SIGSHIFT = 7,
  kNumBids = 8,
};
enum : int { SHARE_NONE = 0, SHARE_INCL = 1, SHARE_EXCL = 2 };

template <int BID> constexpr bool bid_log2() { return BID == BID_SOFTMAX || BID == BID_EXPSHIFT; }
template <int BID> constexpr bool bid_ratio() { return BID >= BID_RELU && BID <= BID_MINSHIFT; }
template <int BID> constexpr bool bid_sigm() { return BID == BID_SIGMOID || BID == BID_SIGSHIFT; }
// rows sum to one: the backward subtracts ghat
template <int BID> constexpr bool bid_normalized() { return BID <= BID_MINSHIFT; }
// the production operator: softmax bids, dilution share
template <int BID, int SHARE> constexpr bool is_production() { return BID == BID_SOFTMAX && SHARE == SHARE_INCL; }

__device__ __forceinline__ float sigmoid_f(float x) { return fast_rcp(1.f + fast_exp2(-kLog2e * x)); }

// numerator f(a) of a ratio bid (a in natural units)
template <int BID>
__device__ __forceinline__ float bid_f(float a) {
  if constexpr (BID == BID_RELU) {
    return fmaxf(a, 0.f);
  } else if constexpr (BID == BID_RELU2) {
    const float r = fmaxf(a, 0.f);
    return r * r;
  } else if constexpr (BID == BID_SOFTPLUS) {
    // max(a, 0) + log(1 + e^-|a|), the stable softplus (kernels_bid.py:219),
    // on the hardware exp2 / log2: 1 + e^-|a| lies in (1, 2]
    return fmaxf(a, 0.f) + kLn2 * fast_log2(1.f + fast_exp2(-kLog2e * fabsf(a)));
  } else {
    return a;                                   // minshift: the row minimum sits in r1
  }
}

// Jacobian numerator u(a) of a ratio bid: jac = u(a) / R
template <int BID>
__device__ __forceinline__ float bid_u(float a) {
  if constexpr (BID == BID_RELU) return a > 0.f ? 1.f : 0.f;
  else if constexpr (BID == BID_RELU2) return 2.f * fmaxf(a, 0.f);
  else if constexpr (BID == BID_SOFTPLUS) return sigmoid_f(a);
  else return 1.f;
}

// Per-row parameters (r0, r1) from the forward's row statistics: rmax, rden as
// the reference stores them (kernels_bid.py:338-349), `window` = the number of
// keys the row sees, `valid` = the row exists.
template <int BID>
__device__ __forceinline__ void bid_row_params(float rmax, float rden, float window, bool valid,
                                               float& r0, float& r1) {
  r1 = 0.f;
  if constexpr (bid_log2<BID>()) {
    r0 = valid ? rmax + __log2f(rden) : INFINITY;
  } else if constexpr (bid_ratio<BID>()) {
    const bool empty = !(rden > 0.f);
    const float rinv = (valid && !empty) ? 1.f / rden : 0.f;
    r0 = rinv;
    if (valid) {
      if (empty) r1 = -1.f / window;
      else if (BID == BID_MINSHIFT) r1 = rmax * rinv;
    }
  } else {
    r0 = valid ? 1.f : 0.f;
  }
}

// p from the raw dot product q.k (`dot`), c = log2(e)/sqrt(D), s = 1/sqrt(D),
// lshift = log2(SHIFT).
template <int BID>
__device__ __forceinline__ float bid_p(float dot, float c, float s, float r0, float r1, float lshift) {
  if constexpr (bid_log2<BID>()) {
    return fast_exp2(fmaf(dot, c, -r0));
  } else if constexpr (bid_ratio<BID>()) {
    // no fma contraction here (__fmul_rn is a plain, contractible product in
    // HIP): the row's minimum must give fl(a r0) - fl(a r0) = 0 exactly
#pragma clang fp contract(off)
    const float a = dot * s;
    return bid_f<BID>(a) * r0 - r1;
  } else {
    // sigshift: sigmoid(a - log SHIFT) = 1 / (1 + 2^(log2 SHIFT - a log2 e)); sigmoid: no shift
    const float off = BID == BID_SIGSHIFT ? lshift : 0.f;
    return r0 * fast_rcp(1.f + fast_exp2(off - dot * c));
  }
}

// dp/da (diagonal part) given p
template <int BID>
__device__ __forceinline__ float bid_jac(float p, float dot, float s, float r0) {
  if constexpr (bid_log2<BID>()) return p;
  else if constexpr (bid_ratio<BID>()) return bid_u<BID>(dot * s) * r0;
  else return p * (1.f - p);
}

}  // namespace dil
