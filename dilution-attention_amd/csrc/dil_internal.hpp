// Host-side declarations shared by the kernel translation units and the C ABI.
#pragma once

#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

namespace dil {

// Negative status codes (positive values are hipError_t).  Mirrored by
// dil_status_string() and by the Python layer.
constexpr int kErrHeadDim = -1;
constexpr int kErrDtype = -2;
constexpr int kErrWorkspace = -3;
constexpr int kErrShape = -4;
constexpr int kErrPrecision = -5;
constexpr int kErrVariant = -6;
constexpr int kErrScratch = -7;

// Operator variant (the reference's kernels_bid ablations): bid function
// 0..7, share mode 0 (none) / 1 (dilution) / 2 (exclusive), and the SHIFT of
// the expshift / sigshift bids.  The production operator is {0, 1, 1}; every
// variant is built for the head dims of the production operator.
struct Variant {
  int bid = 0;
  int share = 1;
  float shift = 1.f;
};
int check_variant(const Variant& v, int head_dim);

inline size_t align_up(size_t bytes) { return (bytes + 255) & ~static_cast<size_t>(255); }

// Kernels that put the slice index on grid y (limited to 65535 blocks) are
// launched once per batch of slices: f(first slice, slices in the batch).
constexpr int64_t kMaxGridY = 65535;
template <typename F>
inline void slice_batches(int64_t n, F&& f) {
  for (int64_t s0 = 0; s0 < n; s0 += kMaxGridY)
    f(s0, static_cast<unsigned>(n - s0 < kMaxGridY ? n - s0 : kMaxGridY));
}

// Brackets one kernel launch with hipEvents on `stream` while kernel timing
// is enabled (dil_timing_enable); a no-op otherwise.  `name` must be a string
// literal: it is kept until the timing is read.
class LaunchTimer {
 public:
  LaunchTimer(const char* name, void* stream);
  ~LaunchTimer();
  LaunchTimer(const LaunchTimer&) = delete;
  LaunchTimer& operator=(const LaunchTimer&) = delete;

 private:
  const char* name_;
  void* stream_;
  void* start_ = nullptr;
  void* stop_ = nullptr;
};

// Launch `expr` (a kernel launch statement) inside a LaunchTimer scope.
#define DIL_TIMED(name, stream, ...) \
  do {                               \
    ::dil::LaunchTimer _dil_t(name, stream); \
    __VA_ARGS__;                     \
  } while (0)

struct DecodeArgs {
  const void* q1;        // (n, D) rows in `q_dtype`, slice stride q_sn elements
  int64_t q_sn;
  const void* k_cache;   // (n, cap, D), slice stride kv_sn elements
  const void* v_cache;
  int64_t kv_sn;
  float* committed;      // (n, cap) fp32, slice stride c_sn
  int64_t c_sn;
  void* out;             // (n, D) in `q_dtype`, slice stride o_sn
  int64_t o_sn;
  void* workspace;
  int64_t workspace_bytes;
  int64_t n, length;     // with dlen: the maximum length (grid and scratch sized for it)
  const int64_t* dlen;   // null, or the live length in device memory (clamped to [0, length])
  int head_dim, dtype;   // dtype: the caches'
  int q_dtype;           // q1's and the output's
  Variant var;
  void* stream;
};

int64_t decode_workspace_bytes(int64_t n, int64_t length, int head_dim);
int decode_step(const DecodeArgs& a);

// Forward over query rows [q0, q0 + C) against keys [0, Tk), Tk = q0 + C.
// Plain forward: q0 = 0, C = Tk = T.  Chunked prefill: q0 = chunk start.
struct ForwardArgs {
  const void* q;         // (n, C, D) rows, slice stride q_sn
  int64_t q_sn;
  const void* k;         // (n, >= Tk, D), slice stride kv_sn
  const void* v;
  int64_t kv_sn;
  int64_t n, C, Tk, q0;
  int head_dim, dtype, prec;   // precision code: 0 fp32, 1 split (tf32), 2 bf16 MFMA operands
  float* out;            // (n, C, D) fp32, slice stride o_sn
  int64_t o_sn;
  float* rmax;           // (n, C) fp32 (log2-domain row max of the scaled affinities)
  float* rden;           // (n, C) fp32 (sum of 2^(a - rmax))
  float* ssum;           // (n, C) fp32 (row sum of shares)
  float* carry;          // (n, ceil(C/32), Tk) fp32 demand checkpoints
  const float* demand_in;  // (n, >= q0) fp32 demand before row q0, or null
  int64_t din_sn;
  float* total;          // (n, Tk) fp32 demand after the last row (may alias demand_in)
  int64_t tot_sn;
  float* pk;             // (n, C, D) fp32 scale * jac @ k (jac = p for softmax bids), or null
  Variant var;
  bool key_pass;         // the key-parallel output pass is requested (read once per call)
  void* workspace;
  int64_t workspace_bytes;
  void* stream;
};

// The key-parallel output pass serves the calls that can take it unless the
// environment sets DILUTION_FORWARD_KEY_PASS=0 (the three-pass forward for
// every call).  Each entry point reads it once and hands the answer to both
// its workspace check and its launch, so a change of the variable between the
// two cannot make them disagree.
inline bool forward_key_pass_requested() {
  const char* e = getenv("DILUTION_FORWARD_KEY_PASS");
  return !(e != nullptr && e[0] == '0' && e[1] == '\0');
}

int64_t forward_workspace_bytes(int64_t n, int64_t C, int64_t Tk, int head_dim, int dtype, int prec,
                                int want_pk, bool key_pass);
// Whether a forward over rows [q0, q0 + C) against keys [0, Tk) takes the
// key-parallel output pass, whose demand checkpoints are an output only (the
// caller may then pass no carry array); the three-pass forward reads them.
bool forward_takes_key_pass(int64_t C, int64_t Tk, int64_t q0, int head_dim, int prec, const Variant& var,
                            bool key_pass);
int forward(const ForwardArgs& a);

struct BackwardArgs {
  const void* q;         // (n, T, D) each, contiguous slices of T*D
  const void* k;
  const void* v;
  const void* dout;      // (n, T, D) in dout_dtype
  const float* out;      // (n, T, D) fp32 forward output
  const float* rmax;     // (n, T)
  const float* rden;
  const float* ssum;
  const float* carry;    // (n, ceil(T/32), T)
  const float* pk;       // (n, T, D)
  Variant var;
  void* dq;              // (n, T, D) each in grad_dtype
  void* dk;
  void* dv;
  int64_t n, T;
  int head_dim, dtype, dout_dtype, grad_dtype, prec;   // prec as in ForwardArgs
  void* workspace;
  int64_t workspace_bytes;
  void* stream;
};

int64_t backward_workspace_bytes(int64_t n, int64_t T, int head_dim, int dtype, int prec);
int backward(const BackwardArgs& a);

// The ablation variants of one bid function (any share mode and head_dim);
// each bid is built in its own object from dil_variants.hip.
template <int BID> int forward_bid(const ForwardArgs& a);
template <int BID> int backward_bid(const BackwardArgs& a);
template <int BID> int decode_bid(const DecodeArgs& a);

}  // namespace dil
