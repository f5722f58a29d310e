# integrate_worker.awk — test infrastructure: streams the reference's
# expert_node_v2/worker.cc to the compiler with the one-branch worker-loop edit
# that integrating the AMD plugin's whole-layer message takes, so the node
# harness runs the reference's own RunGpuWorkerLoopV2 with that edit and
# nothing else changed.  The output goes to a pipe, never to a file.
#
# The edit (worker.cc:256-264 closes the connection on every type but
# InferRequest):
#   * after the include of expert_node_v2/expert_registry_v2.h, the plugin's
#     handler header;
#   * before the InferRequest check, a branch for msg_type 42 that calls
#     HandleMoeLayerRequestAmdV2 and keeps the connection on success.
# Fails (exit 1) unless each anchor occurs exactly once.
BEGIN { inc = 0; br = 0 }
/^#include "expert_node_v2\/expert_registry_v2\.h"/ {
    print
    print "#include \"expert_node_v2/backend/amd/moe_layer_worker_amd_v2.h\""
    inc++
    next
}
/if \(msg_type != common::MsgType::InferRequest\) \{/ {
    print "            if (req.msg_type == expert_node_v2::kMsgMoeLayerRequestV2) {     // 42"
    print "                if (!expert_node_v2::HandleMoeLayerRequestAmdV2(fd, ctx, req, req_body)) break;"
    print "                continue;"
    print "            }"
    br++
}
{ print }
END {
    if (inc != 1 || br != 1) {
        printf "integrate_worker.awk: anchors found %d (include), %d (branch); expected 1 each\n", inc, br > "/dev/stderr"
        exit 1
    }
}
