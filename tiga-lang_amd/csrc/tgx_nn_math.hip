// The edge-MLP kernels and entry points of tgx_nn.hip built with the second
// set of component-wise functions (exp, log, abs, sin, cos, the powers) and
// LayerNorm, as the tgx_edge_mlp_*_math functions; tgx_nn_common.h says why
// the set has kernels of its own.
#define TGX_NN_MATH 1
#include "tgx_nn.hip"
