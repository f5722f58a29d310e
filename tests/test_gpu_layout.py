"""Gate/up weights in CX_LAYOUT_TILE16 (cx_upload_matrix_tiled, and what
cx_gen_expert writes) against the same bytes row-major: the resident bytes
read back equal, and every kernel path that reads gate/up gives bit-identical
outputs (one expert at 1..40 tokens; layers mixing both layouts through the
one-token pipeline, the decode pipeline, the grouped prefill GEMM and the
LDS-ring GEMM)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _host_expert(rng, H, I, blk=128):
    def mat(r, c):
        w = rng.integers(0, 0x7E, (r, c), dtype=np.uint8)
        w ^= rng.integers(0, 2, (r, c), dtype=np.uint8) << 7          # both signs
        w.ravel()[rng.integers(0, r * c, 64)] = 0x7F                      # non-finite codes: canonicalised
        w.ravel()[rng.integers(0, r * c, 64)] = 0xFF
        return w
    def sc(r, c):
        return rng.uniform(5e-4, 2e-3, ((r + blk - 1) // blk, (c + blk - 1) // blk)).astype(np.float32)
    return dict(w_up=mat(I, H), s_up=sc(I, H), w_gate=mat(I, H), s_gate=sc(I, H),
                w_down=mat(H, I), s_down=sc(H, I))


def _upload(ex, tiled, blk=128):
    from constellation_amd.engine import Expert
    return Expert.upload(0, ex["w_up"], ex["s_up"], ex["w_gate"], ex["s_gate"], ex["w_down"],
                         ex["s_down"], row_block=blk, col_block=blk, tiled=tiled)


def _canon(w):
    w = w.copy()
    w[(w & 0x7F) == 0x7F] -= 1
    return w


def test_tiled_upload_reads_back_and_runs_like_rows(gpu):
    print("[layout] tiled upload, one expert", flush=True)
    rng = np.random.default_rng(7)
    H, I = 7168, 2048
    ex = _host_expert(rng, H, I)
    rows, tile = _upload(ex, False), _upload(ex, True)
    try:
        assert rows.desc.gu_layout == 0 and tile.desc.gu_layout == 1
        a, b = rows.download(), tile.download()
        for k in ("w_up", "w_gate", "w_down"):
            assert np.array_equal(b[k], _canon(ex[k])), k
            assert np.array_equal(a[k], b[k]), k
        for k in ("s_up", "s_gate", "s_down"):
            assert np.array_equal(a[k], b[k]), k
        for T in (1, 3, 5, 17, 40):
            x = gpu.gen_normal(8, T, (T, H), 1.0, torch.bfloat16)
            ya, yfa = gpu.expert_run(rows, x, want_f32=True)
            yb, yfb = gpu.expert_run(tile, x, want_f32=True)
            torch.cuda.synchronize()
            assert torch.equal(yfa.view(torch.int32), yfb.view(torch.int32)), T
            assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), T
    finally:
        rows.free()
        tile.free()


@pytest.mark.parametrize("H,I,blk,Ts", [(7168, 2048, 128, (1, 5, 40)), (1024, 512, 64, (1, 4, 20))])
def test_tiled_fp16_input_and_generic_path(gpu, H, I, blk, Ts):
    """fp16 activations (the F16 instances of every gate/up body) at full
    size, and 64 x 64 scale blocks, which only the generic kernels take
    (gu_elem_off per element): tiled and row-major give the same bits."""
    print(f"[layout] fp16 / generic H={H} I={I} blk={blk}", flush=True)
    rng = np.random.default_rng(blk)
    ex = _host_expert(rng, H, I, blk)
    rows, tile = _upload(ex, False, blk), _upload(ex, True, blk)
    try:
        assert tile.desc.gu_layout == 1
        for T in Ts:
            for dt in (torch.float16, torch.bfloat16):
                x = gpu.gen_normal(9, T, (T, H), 1.0, torch.float32).to(dt)
                ya, yfa = gpu.expert_run(rows, x, want_f32=True)
                yb, yfb = gpu.expert_run(tile, x, want_f32=True)
                torch.cuda.synchronize()
                assert torch.equal(yfa.view(torch.int32), yfb.view(torch.int32)), (T, dt)
                assert torch.equal(ya.view(torch.int16), yb.view(torch.int16)), (T, dt)
    finally:
        rows.free()
        tile.free()


def test_generated_expert_is_tiled_and_matches_row_major_upload(gpu):
    """cx_gen_expert writes up and gate tiled; the same bytes uploaded
    row-major run identically."""
    print("[layout] generated expert", flush=True)
    from constellation_amd.engine import Expert
    g = Expert.generate(0, 31, 0x3100)
    try:
        assert g.desc.gu_layout == 1
        ex = g.download()
        r = Expert.upload(0, ex["w_up"], ex["s_up"], ex["w_gate"], ex["s_gate"], ex["w_down"],
                          ex["s_down"], tiled=False)
        try:
            x = gpu.gen_normal(32, 1, (4, 7168), 1.0, torch.bfloat16)
            ya = gpu.expert_run(g, x)
            yb = gpu.expert_run(r, x)
            torch.cuda.synchronize()
            assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
        finally:
            r.free()
    finally:
        g.free()


@pytest.mark.parametrize("T,K,E", [(1, 8, 32), (5, 8, 32), (16, 8, 32), (70, 8, 32), (200, 4, 4)])
def test_layer_mixing_layouts_equals_row_major_layer(gpu, T, K, E):
    """Routes given (cx_moe): T = 1 the one-token down + combine, T <= 16 the
    decode pipeline, 70 the grouped GEMM, 200 x 4 routes over 4 experts the
    LDS-ring GEMM (>= 128 pairs per expert).  Experts alternate tiled and
    row-major; the reference layer holds the same bytes all row-major."""
    print(f"[layout] layer T={T} K={K} E={E}", flush=True)
    from constellation_amd.engine import Layer
    rng = np.random.default_rng(T)
    H, I = 1024, 512
    host = [_host_expert(rng, H, I) for _ in range(E + 1)]
    mixed = [_upload(ex, i % 2 == 0) for i, ex in enumerate(host)]
    plain = [_upload(ex, False) for ex in host]
    la = Layer(gpu, mixed[:E], mixed[E])
    lb = Layer(gpu, plain[:E], plain[E])
    try:
        x = gpu.gen_normal(40 + T, 1, (T, H), 1.0, torch.bfloat16)
        ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
        wts = rng.uniform(0.05, 1.0, ids.shape).astype(np.float32)
        ids_t, wts_t = torch.from_numpy(ids).cuda(), torch.from_numpy(wts).cuda()
        ya, yfa = gpu.moe(la, x, ids_t, wts_t, want_f32=True)
        yb, yfb = gpu.moe(lb, x, ids_t, wts_t, want_f32=True)
        gpu.sync()
        assert torch.equal(yfa.view(torch.int32), yfb.view(torch.int32))
        assert torch.equal(ya.view(torch.int16), yb.view(torch.int16))
    finally:
        la.close()
        lb.close()
        for e in mixed + plain:
            e.free()
