// The 64-wide backward passes of tgx_nn_wide.hip built with the second set
// of component-wise functions, for tgx_nn_math.hip.
#define TGX_NN_MATH 1
#include "tgx_nn_wide.hip"
