// One-launch decode routers for sigmoid scoring: the kernels of
// launch_topk_permute / launch_gate_topk_permute (router.h), instantiated in
// a translation unit of their own so the build compiles the scoring modes in
// parallel.
#include "router.h"

namespace lmoe {

template int launch_topk_permute<LMOE_SCORING_SIGMOID>(const RouterPermuteArgs&, hipStream_t);
template int launch_gate_topk_permute<LMOE_SCORING_SIGMOID>(const RouterPermuteArgs&, hipStream_t);

}  // namespace lmoe

LMOE_FLAGS_UNIT(router_sigmoid)
