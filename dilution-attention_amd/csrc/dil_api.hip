// extern "C" entry points of libdilution_hip.so (declared in include/dilution_hip.h).
// Argument checks that need no device access happen here; every launch is
// asynchronous on the caller's stream.
#include <hip/hip_runtime.h>

#include "../../include/dilution_hip.h"
#include "dil_internal.hpp"
#include "dil_variant.hpp"

namespace {

bool valid_head_dim(int d) { return d == 16 || d == 32 || d == 64 || d == 128 || d == 256; }
// head_dim 256 runs with bf16 operands only: the fp32 and split-operand tiles
// of the row-parallel output pass exceed the 160 KB of LDS at that width
bool valid_head_dim(int d, int precision) { return valid_head_dim(d) && (d < 256 || precision == 2); }
bool valid_dtype(int t) { return t == 0 || t == 1 || t == 2; }
bool valid_precision(int p) { return p == 0 || p == 1 || p == 2; }

// True when every pointer is non-null (a required argument).
template <typename... Ps>
bool all_set(const Ps*... ps) {
  return ((ps != nullptr) && ...);
}

}  // namespace

namespace dil {

int check_variant(const Variant& v, int head_dim) {
  if (v.bid < 0 || v.bid >= kNumBids || v.share < SHARE_NONE || v.share > SHARE_EXCL || !(v.shift > 0.f))
    return kErrVariant;
  (void)head_dim;                            // every variant is built for every valid head_dim
  return 0;
}

}  // namespace dil

extern "C" {

int dil_abi_version(void) { return 4; }

const char* dil_status_string(int status) {
  switch (status) {
    case 0: return "success";
    case dil::kErrHeadDim:
      return "head_dim must be one of 16, 32, 64, 128, or 256 with bf16 operands (the bid / share "
             "variants: 16-128)";
    case dil::kErrDtype: return "unsupported dtype code";
    case dil::kErrWorkspace: return "workspace smaller than the size query returned";
    case dil::kErrShape: return "invalid shape or length";
    case dil::kErrPrecision: return "dot_precision must be one of ieee, tf32, bf16";
    case dil::kErrVariant:
      return "operator variant out of range (bid 0-7, share 0-2, shift > 0)";
    case dil::kErrScratch:
      return "the call needs more scratch than dil_decode_step_noalloc holds "
             "(DIL_NOALLOC_SCRATCH_BYTES); use dil_decode_step with a workspace";
    default: break;
  }
  if (status > 0) return hipGetErrorString(static_cast<hipError_t>(status));
  return "unknown status";
}

int64_t dil_decode_workspace_bytes(int64_t n, int64_t length, int head_dim) {
  return dil::decode_workspace_bytes(n, length, head_dim);
}

int dil_decode_step_variant(const void* q1, const void* k_cache, const void* v_cache,
                            float* committed, void* out, int64_t n, int64_t capacity,
                            int64_t length, int head_dim, int dtype, int q_dtype, int bid,
                            int share, float shift, void* workspace, int64_t workspace_bytes,
                            void* stream) {
  if (!valid_head_dim(head_dim)) return dil::kErrHeadDim;
  if (!valid_dtype(dtype) || !valid_dtype(q_dtype)) return dil::kErrDtype;
  if (n < 1 || length < 1 || length > capacity) return dil::kErrShape;
  if (!all_set(q1, k_cache, v_cache, static_cast<const void*>(committed), static_cast<const void*>(out),
               static_cast<const void*>(workspace)))
    return dil::kErrShape;
  if (workspace_bytes < dil::decode_workspace_bytes(n, length, head_dim)) return dil::kErrWorkspace;
  dil::DecodeArgs a{};
  a.q1 = q1;
  a.q_sn = head_dim;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_sn = capacity * head_dim;
  a.committed = committed;
  a.c_sn = capacity;
  a.out = out;
  a.o_sn = head_dim;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.n = n;
  a.length = length;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.q_dtype = q_dtype;
  a.var = dil::Variant{bid, share, shift};
  a.stream = stream;
  return dil::decode_step(a);
}

int dil_decode_step(const void* q1, const void* k_cache, const void* v_cache, float* committed,
                    void* out, int64_t n, int64_t capacity, int64_t length, int head_dim,
                    int dtype, int q_dtype, void* workspace, int64_t workspace_bytes, void* stream) {
  return dil_decode_step_variant(q1, k_cache, v_cache, committed, out, n, capacity, length,
                                 head_dim, dtype, q_dtype, 0, 1, 1.f, workspace, workspace_bytes,
                                 stream);
}

int dil_decode_step_dlen(const void* q1, const void* k_cache, const void* v_cache, float* committed,
                         void* out, int64_t n, int64_t capacity, const int64_t* length,
                         int64_t max_length, int head_dim, int dtype, int q_dtype, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  if (!valid_head_dim(head_dim)) return dil::kErrHeadDim;
  if (!valid_dtype(dtype) || !valid_dtype(q_dtype)) return dil::kErrDtype;
  if (n < 1 || max_length < 1 || max_length > capacity) return dil::kErrShape;
  if (!all_set(q1, k_cache, v_cache, static_cast<const void*>(committed), static_cast<const void*>(out),
               static_cast<const void*>(length), static_cast<const void*>(workspace)))
    return dil::kErrShape;
  if (workspace_bytes < dil::decode_workspace_bytes(n, max_length, head_dim)) return dil::kErrWorkspace;
  dil::DecodeArgs a{};
  a.q1 = q1;
  a.q_sn = head_dim;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_sn = capacity * head_dim;
  a.committed = committed;
  a.c_sn = capacity;
  a.out = out;
  a.o_sn = head_dim;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.n = n;
  a.length = max_length;
  a.dlen = length;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.q_dtype = q_dtype;
  a.var = dil::Variant{0, 1, 1.f};
  a.stream = stream;
  return dil::decode_step(a);
}

int64_t dil_forward_workspace_bytes(int64_t n, int64_t seq, int head_dim, int dtype,
                                    int precision, int want_pk) {
  return dil::forward_workspace_bytes(n, seq, seq, head_dim, dtype, precision, want_pk,
                                      dil::forward_key_pass_requested());
}

int dil_forward_variant(const void* q, const void* k, const void* v, int64_t n, int64_t seq,
                        int head_dim, int dtype, int precision, int bid, int share, float shift,
                        float* out, float* rmax, float* rden, float* ssum, float* carry,
                        float* committed_total, float* pk, void* workspace, int64_t workspace_bytes,
                        void* stream) {
  if (!valid_head_dim(head_dim, precision)) return dil::kErrHeadDim;
  if (!valid_dtype(dtype)) return dil::kErrDtype;
  if (!valid_precision(precision)) return dil::kErrPrecision;
  if (n < 1 || seq < 1) return dil::kErrShape;
  // carry may be null when the call takes the key pass (dil::forward checks)
  if (!all_set(q, k, v, static_cast<const void*>(out), static_cast<const void*>(rmax),
               static_cast<const void*>(rden), static_cast<const void*>(ssum),
               static_cast<const void*>(committed_total), static_cast<const void*>(workspace)))
    return dil::kErrShape;
  const bool key_pass = dil::forward_key_pass_requested();
  if (workspace_bytes <
      dil::forward_workspace_bytes(n, seq, seq, head_dim, dtype, precision, pk != nullptr, key_pass))
    return dil::kErrWorkspace;
  dil::ForwardArgs a{};
  a.key_pass = key_pass;
  a.q = q;
  a.q_sn = seq * head_dim;
  a.k = k;
  a.v = v;
  a.kv_sn = seq * head_dim;
  a.n = n;
  a.C = seq;
  a.Tk = seq;
  a.q0 = 0;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.prec = precision;
  a.out = out;
  a.o_sn = seq * head_dim;
  a.rmax = rmax;
  a.rden = rden;
  a.ssum = ssum;
  a.carry = carry;
  a.demand_in = nullptr;
  a.din_sn = 0;
  a.total = committed_total;
  a.tot_sn = seq;
  a.pk = pk;
  a.var = dil::Variant{bid, share, shift};
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  return dil::forward(a);
}

int dil_forward(const void* q, const void* k, const void* v, int64_t n, int64_t seq,
                int head_dim, int dtype, int precision, float* out, float* rmax, float* rden,
                float* ssum, float* carry, float* committed_total, float* pk, void* workspace,
                int64_t workspace_bytes, void* stream) {
  return dil_forward_variant(q, k, v, n, seq, head_dim, dtype, precision, 0, 1, 1.f, out, rmax,
                             rden, ssum, carry, committed_total, pk, workspace, workspace_bytes,
                             stream);
}

int dil_forward_key_pass(int64_t chunk, int64_t start, int head_dim, int dtype, int precision) {
  if (!valid_head_dim(head_dim) || !valid_dtype(dtype) || !valid_precision(precision) || chunk < 1 ||
      start < 0)
    return 0;
  return dil::forward_takes_key_pass(chunk, start + chunk, start, head_dim, precision, dil::Variant{},
                                     dil::forward_key_pass_requested())
             ? 1
             : 0;
}

int64_t dil_prefill_workspace_bytes(int64_t n, int64_t chunk, int64_t start, int head_dim,
                                    int dtype, int precision) {
  return dil::forward_workspace_bytes(n, chunk, start + chunk, head_dim, dtype, precision, 0,
                                      dil::forward_key_pass_requested());
}

int dil_prefill_chunk(const void* q_chunk, const void* k_cache, const void* v_cache, int64_t n,
                      int64_t chunk, int64_t start, int64_t capacity, int head_dim, int dtype,
                      int precision, float* committed, float* out, float* rmax, float* rden,
                      float* ssum, float* carry, void* workspace, int64_t workspace_bytes,
                      void* stream) {
  if (!valid_head_dim(head_dim, precision)) return dil::kErrHeadDim;
  if (!valid_dtype(dtype)) return dil::kErrDtype;
  if (!valid_precision(precision)) return dil::kErrPrecision;
  if (n < 1 || chunk < 1 || start < 0 || start + chunk > capacity) return dil::kErrShape;
  // carry may be null when the chunk takes the key pass (dil::forward checks)
  if (!all_set(q_chunk, k_cache, v_cache, static_cast<const void*>(committed),
               static_cast<const void*>(out), static_cast<const void*>(rmax),
               static_cast<const void*>(rden), static_cast<const void*>(ssum),
               static_cast<const void*>(workspace)))
    return dil::kErrShape;
  const bool key_pass = dil::forward_key_pass_requested();
  if (workspace_bytes <
      dil::forward_workspace_bytes(n, chunk, start + chunk, head_dim, dtype, precision, 0, key_pass))
    return dil::kErrWorkspace;
  dil::ForwardArgs a{};
  a.key_pass = key_pass;
  a.q = q_chunk;
  a.q_sn = chunk * head_dim;
  a.k = k_cache;
  a.v = v_cache;
  a.kv_sn = capacity * head_dim;
  a.n = n;
  a.C = chunk;
  a.Tk = start + chunk;
  a.q0 = start;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.prec = precision;
  a.out = out;
  a.o_sn = chunk * head_dim;
  a.rmax = rmax;
  a.rden = rden;
  a.ssum = ssum;
  a.carry = carry;
  a.demand_in = committed;
  a.din_sn = capacity;
  a.total = committed;
  a.tot_sn = capacity;
  a.pk = nullptr;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  return dil::forward(a);
}

int64_t dil_backward_workspace_bytes(int64_t n, int64_t seq, int head_dim, int dtype,
                                     int precision) {
  return dil::backward_workspace_bytes(n, seq, head_dim, dtype, precision);
}

int dil_backward_variant(const void* q, const void* k, const void* v, const void* dout,
                         const float* out, const float* rmax, const float* rden,
                         const float* ssum, const float* carry, const float* pk, int64_t n,
                         int64_t seq, int head_dim, int dtype, int dout_dtype, int grad_dtype,
                         int precision, int bid, int share, float shift, void* dq, void* dk,
                         void* dv, void* workspace, int64_t workspace_bytes, void* stream) {
  if (!valid_head_dim(head_dim, precision)) return dil::kErrHeadDim;
  if (!valid_dtype(dtype) || !valid_dtype(dout_dtype) || !valid_dtype(grad_dtype))
    return dil::kErrDtype;
  if (!valid_precision(precision)) return dil::kErrPrecision;
  if (n < 1 || seq < 1) return dil::kErrShape;
  if (!all_set(q, k, v, dout, static_cast<const void*>(out), static_cast<const void*>(rmax),
               static_cast<const void*>(rden), static_cast<const void*>(ssum),
               static_cast<const void*>(carry), static_cast<const void*>(pk), dq, dk, dv,
               static_cast<const void*>(workspace)))
    return dil::kErrShape;
  if (workspace_bytes < dil::backward_workspace_bytes(n, seq, head_dim, dtype, precision))
    return dil::kErrWorkspace;
  dil::BackwardArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.dout = dout;
  a.out = out;
  a.rmax = rmax;
  a.rden = rden;
  a.ssum = ssum;
  a.carry = carry;
  a.pk = pk;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.n = n;
  a.T = seq;
  a.head_dim = head_dim;
  a.dtype = dtype;
  a.dout_dtype = dout_dtype;
  a.grad_dtype = grad_dtype;
  a.prec = precision;
  a.var = dil::Variant{bid, share, shift};
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  return dil::backward(a);
}

int dil_backward(const void* q, const void* k, const void* v, const void* dout,
                 const float* out, const float* rmax, const float* rden, const float* ssum,
                 const float* carry, const float* pk, int64_t n, int64_t seq, int head_dim,
                 int dtype, int dout_dtype, int grad_dtype, int precision, void* dq, void* dk,
                 void* dv, void* workspace, int64_t workspace_bytes, void* stream) {
  return dil_backward_variant(q, k, v, dout, out, rmax, rden, ssum, carry, pk, n, seq, head_dim,
                              dtype, dout_dtype, grad_dtype, precision, 0, 1, 1.f, dq, dk, dv,
                              workspace, workspace_bytes, stream);
}

}  // extern "C"
