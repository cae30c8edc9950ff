"""torch.library registration (CPU only: FakeTensor tracing, no kernel runs).

Every HIP launch of the package is a custom op torch.ops.fsi.<name>; these tests
check that the expected ops exist, that their fake implementations give the
shapes and dtypes the real launches produce, and that a routed decode step
traces into a graph whose nodes are the fsi ops (what torch.compile / export
see)."""
import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

EXPECTED = {
    "additive_context", "additive_context_bwd", "block_scores", "block_scores_bwd", "block_sparse_linear",
    "blockwise_matmul", "decode_attention", "decode_route", "decode_step_attention", "dense_block_targets", "distill_kl", "distill_kl_bwd",
    "index_rms_norm", "index_rms_norm_bwd", "kv_page_pool", "kv_read", "kv_write", "masked_softmax",
    "masked_softmax_bwd", "mlp_router", "pattention", "pattention_pack", "pattention_packed", "pool_kv",
    "pool_kv_bwd", "route_from_scores", "score_and_route", "sparse_attention", "sram_indexer_attention", "swiglu",
    "swiglu_bwd", "tile_route",
}


@pytest.fixture(scope="module")
def ops(fsi):
    return torch.ops.fsi


def test_every_launch_is_registered(ops):
    have = {n for n in dir(ops) if not n.startswith("_") and n != "name"}
    assert EXPECTED <= have, EXPECTED - have


def _fake(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, dtype=dtype, device="cuda")


def test_fake_shapes(ops):
    with FakeTensorMode():
        s = _fake(2, 8, 32, dtype=torch.float32)
        idx, cnt = ops.route_from_scores(s, True, 2, 0.9, 0, 4, 6, None, None, None, 0)
        assert idx.shape == (2, 8, 6) and idx.dtype == torch.int32 and cnt.shape == (2, 8)
        i2, c2, mass = ops.score_and_route(_fake(2, 5, 16), _fake(1, 40, 16), False, 0, 0.9, 0, 8, 8, True)
        assert i2.shape == (2, 5, 8) and mass.shape == (2, 5) and mass.dtype == torch.float32
        x = _fake(64, 4096)
        y = ops.pattention(x, _fake(14336, 4096), _fake(14336, 4096), _fake(14336, 4096), _fake(64, dtype=torch.int32),
                           64, 0, 1, False)
        assert y.shape == (64, 4096) and y.dtype == torch.bfloat16
        y = ops.pattention_packed(x, _fake(1 << 20, dtype=torch.uint8), None, 14336, 4096, 64, 1)
        assert y.shape == (64, 4096)
        a, sc = ops.mlp_router(x, _fake(16, 4096), _fake(224, 16), 8, 56, 1.0, True)
        assert a.shape == (64,) and a.dtype == torch.int32 and sc.shape == (224,)
        q = _fake(2, 8, 256, 64)
        kv = _fake(2, 2, 256, 64)
        o = ops.sparse_attention(q, kv, kv, _fake(2, 4, 3, dtype=torch.int32), _fake(2, 4, dtype=torch.int32), 3, 64,
                                 0, 64, 0.125)
        assert o.shape == q.shape and o.transpose(1, 2).is_contiguous()
        pages, counts, ctx = ops.decode_route(_fake(4, 16), _fake(4, 10, 16, dtype=torch.float32), _fake(4, 10, 16),
                                              None, 700, 64, 256, 10, 0.9, 2, 6, 6, True)
        assert pages.shape == (4, 6) and counts.shape == (4,) and ctx.shape == (4, 16)
        q3 = _fake(4, 8, 128)
        o = ops.decode_attention(q3, _fake(40, 2, 64, 128), _fake(40, 2, 64, 128), _fake(4, 10, dtype=torch.int32),
                                 10, 40, 640, 64, 2, None, 700, 256, None, None, 0, 0.1)
        assert o.shape == q3.shape
        lin = ops.block_sparse_linear(_fake(10, 256), _fake(512, 256), None, _fake(3, dtype=torch.int32), 64)
        assert lin.shape == (10, 512)
        mask, probs, need = ops.tile_route(_fake(7, 48, dtype=torch.float32), 0.5, 2, 3)
        assert mask.shape == (3, 48) and mask.dtype == torch.uint8 and probs.shape == (7, 48) and need.shape == (7,)
        out, sel = ops.sram_indexer_attention(_fake(2, 4, 64, 32, dtype=torch.float16),
                                              _fake(2, 4, 64, 32, dtype=torch.float16),
                                              _fake(2, 4, 64, 32, dtype=torch.float16),
                                              _fake(2, 4, 16, dtype=torch.float16), _fake(2, 4, 16, dtype=torch.float16),
                                              0.17, 0.8, 2, 16, True)
        assert out.shape == (2, 4, 64, 32) and sel.shape == (2, 4, 2) and sel.dtype == torch.int32
        loss, n = ops.distill_kl(_fake(2, 4, 9, dtype=torch.float32), _fake(2, 4, 9, dtype=torch.float32), 0, None,
                                 1.0)
        assert loss.shape == () and n.shape == (1,)


def test_decode_step_traces_to_fsi_ops(fsi):
    """A routed decode step (router -> packed Pattention) traced with fake
    tensors: the graph's call nodes are the two fsi ops."""
    buf_bytes = 1 << 20

    def step(x, wq, keys, buf):
        active = torch.ops.fsi.mlp_router(x, wq, keys, 8, 56, 1.0, False)[0]
        return torch.ops.fsi.pattention_packed(x, buf, active, 14336, 4096, 64, 1)

    with FakeTensorMode():
        args = (_fake(64, 4096), _fake(16, 4096), _fake(224, 16), _fake(buf_bytes, dtype=torch.uint8))
        gm = make_fx(step, tracing_mode="fake")(*args)
    targets = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert any("fsi.mlp_router" in t for t in targets) and any("fsi.pattention_packed" in t for t in targets)
