// Backward of the dilution-attention operator (in progress).
#include "dil_common.hpp"
#include "dil_internal.hpp"

namespace dil {

int64_t backward_workspace_bytes(int64_t, int64_t, int, int, int) { return 0; }
int backward(const BackwardArgs&) { return kErrShape; }

}  // namespace dil
