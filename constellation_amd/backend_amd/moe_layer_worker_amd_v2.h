// moe_layer_worker_amd_v2.h — worker-side handler of the whole-layer message
// (MoeLayerRequest, msg_type 42 -> MoeLayerResponse 43; byte layout in
// include/cx_moe.h).  No counterpart in the reference: RunGpuWorkerLoopV2
// (expert_node_v2/worker.cc:256-264) closes the connection on every type but
// InferRequest.  The integration adds one branch there that calls
// HandleMoeLayerRequestAmdV2, the way the loop calls HandleInferRequest
// (worker.cc:83-140).
#pragma once

#include <cstdint>
#include <string>

#include "common/protocol.h"
#include "expert_node_v2/worker.h"

namespace expert_node_v2 {

constexpr std::uint16_t kMsgMoeLayerRequestV2 = 42;
constexpr std::uint16_t kMsgMoeLayerResponseV2 = 43;

// Registry ids.  Routed expert i of layer L is L * experts_per_layer + i, the
// server's global id (server/expert_placement.py:4-25).  A layer's shared
// expert is loaded like any expert, under SharedExpertIdV2(L), above every
// routed id.
constexpr std::int32_t kSharedExpertIdBaseV2 = 1 << 30;
inline std::int32_t SharedExpertIdV2(std::int32_t layer_id) {
    return kSharedExpertIdBaseV2 + layer_id;
}

// Runs one MoeLayerRequest body received on a worker connection and sends the
// MoeLayerResponse with the request's request_id.  The layer's experts on this
// worker are looked up under the state's shared lock, as HandleInferRequest
// does; a local id with no resident expert here answers status 2, one outside
// [0, experts_per_layer) status 1.  The workspace must be the AMD one.
// Returns false when the body does not decode or the send fails; the worker
// loop then closes the connection, as it does for a bad InferRequest.
bool HandleMoeLayerRequestAmdV2(int fd, GpuWorkerContextV2* ctx, const common::MsgHeader& req,
                                const std::string& req_body, int experts_per_layer = 256);

}  // namespace expert_node_v2
