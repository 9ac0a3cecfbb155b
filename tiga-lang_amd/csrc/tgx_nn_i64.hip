// The int64_t-indexed edge-MLP kernels of tgx_nn.hip (compiled apart from
// the int32_t ones so the two build in parallel).
#define TGX_NN_INDEX 64
#include "tgx_nn.hip"
