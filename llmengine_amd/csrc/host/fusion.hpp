// fusion.hpp -- fused launches the HipExecutor substitutes for node groups
// (internal to the host runtime).
#pragma once

#include <unordered_map>
#include <vector>

#include "minillm_hip/runtime.h"

namespace minillm::detail {

// The tiled copy of `raw` made for an [N, K] weight, or nullptr.
const uint8_t* tiled_copy_of(const TiledWeights* tiled, const void* raw, int64_t N, int64_t K);

// One Linear node on 16-row tiles (mle_q8_0_linear_tiled): its weight's tiled
// copy in `tiled` (may be null), or the weight itself when it was re-tiled in
// place.  Returns false (nothing launched) when the node's operands do not
// validate or its weight has neither; the node then runs through its registered
// kernel, which reports the reference's errors.
expected<bool, Status> run_tiled_linear(const Node& node, RuntimeContext& ctx,
                                        const TiledWeights* tiled);

// Linear(gate) + Linear(up) + SwiGLU as one mle_q8_0_linear_swiglu launch
// (the _tiled one when both weights are tiled, by a copy in `tiled` or in
// place; *used_tiled says which ran).  Returns false
// (nothing launched) when the bound tensors do not fit the fused kernel (then
// the nodes run one by one and report their own errors).
expected<bool, Status> run_fused_swiglu(const Node& gate, const Node& up, const Node& sw,
                                        RuntimeContext& ctx,
                                        const TiledWeights* tiled = nullptr,
                                        bool* used_tiled = nullptr);

// 2 or 3 Linear nodes on one input as one mle_q8_0_linear_multi launch (the
// _tiled one when `tiled` holds copies of every weight); same return convention.
expected<bool, Status> run_fused_multi(const std::vector<const Node*>& nodes,
                                       RuntimeContext& ctx,
                                       const TiledWeights* tiled = nullptr,
                                       bool* used_tiled = nullptr);

}  // namespace minillm::detail
