"""cx_moe_layer under HIP graph capture, for serving loops that replay a
captured decode step.

The layer call's device work is kernel launches on the caller's stream only
(no memset, copy or allocation once its context buffers have grown to the
call's size, which the eager warm-up call does).  One call is captured on a
side stream, then replayed three times on new activations written into the
captured input buffer, with eager calls and synchronisations between the
replays; every replay's output, fp32 output, routes and weights equal an
eager call's on the same inputs bit for bit.  T = 1 takes the one-token
pipeline (selection inside the routed gate/up launch, down + combine in one
launch), T = 16 the staged decode pipeline.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T", [1, 16])
def test_moe_layer_graph_replays_equal_eager(gpu, T):
    from constellation_amd.engine import Expert, Layer
    print(f"[graph] moe_layer T={T}", flush=True)
    E, H, I = 256, 1024, 512
    experts = [Expert.generate(0, 120, 0x2000 + 4 * e, hidden=H, inter=I) for e in range(E)]
    sh = Expert.generate(0, 120, 0x2000 + 4 * E, hidden=H, inter=I)
    layer = Layer(gpu, experts, sh)
    try:
        w_r = gpu.gen_normal(121, 1, (E, H), 0.02, torch.bfloat16)
        bias = gpu.gen_normal(121, 2, (E,), 0.01, torch.float32)
        xs = [gpu.gen_normal(122, 0x10 + i, (T, H), 1.0, torch.bfloat16) for i in range(4)]
        x = xs[0].clone()

        def outs():
            return (torch.empty((T, H), dtype=torch.bfloat16, device="cuda"),
                    torch.empty((T, H), dtype=torch.float32, device="cuda"),
                    torch.empty((T, 8), dtype=torch.int32, device="cuda"),
                    torch.empty((T, 8), dtype=torch.float32, device="cuda"))

        def call(inp, o):
            gpu.moe_layer(layer, inp, w_r, bias, n_group=8, topk_group=4, top_k=8, out=o)

        cap, ref = outs(), outs()
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):
            call(x, cap)  # eager warm-up on the captured buffers
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
            call(x, cap)
        torch.cuda.synchronize()
        for i in range(1, 4):
            x.copy_(xs[i])
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            call(xs[i], ref)
            torch.cuda.synchronize()
            assert torch.equal(cap[2], ref[2]), i
            assert torch.equal(cap[3].view(torch.int32), ref[3].view(torch.int32)), i
            assert torch.equal(cap[1].view(torch.int32), ref[1].view(torch.int32)), i
            assert torch.equal(cap[0].view(torch.int16), ref[0].view(torch.int16)), i
        # the replays saw new inputs: the routes of the last differ from the first's
        call(xs[0], ref)
        torch.cuda.synchronize()
        assert not torch.equal(cap[1], ref[1])
        del g
    finally:
        torch.cuda.synchronize()
        layer.close()
        for e in experts:
            e.free()
        sh.free()
