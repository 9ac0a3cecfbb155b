// The int64_t-indexed edge-MLP kernels of tgx_nn_math.hip (the second set
// of functions and LayerNorm).
#define TGX_NN_MATH 1
#define TGX_NN_INDEX 64
#include "tgx_nn.hip"
