// fusion.hpp -- fused launches the HipExecutor substitutes for node groups
// (internal to the host runtime).
#pragma once

#include <vector>

#include "minillm_hip/runtime.h"

namespace minillm::detail {

// Linear(gate) + Linear(up) + SwiGLU as one mle_q8_0_linear_swiglu launch.
// Returns false (nothing launched) when the bound tensors do not fit the fused
// kernel (then the nodes run one by one and report their own errors).
expected<bool, Status> run_fused_swiglu(const Node& gate, const Node& up, const Node& sw,
                                        RuntimeContext& ctx);

// 2 or 3 Linear nodes on one input as one mle_q8_0_linear_multi launch; same
// return convention.
expected<bool, Status> run_fused_multi(const std::vector<const Node*>& nodes,
                                       RuntimeContext& ctx);

}  // namespace minillm::detail
