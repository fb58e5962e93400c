"""GPU tests of the context runtime around the products: products recorded
under stream capture (HIP graphs) and replayed, stream changes between
products, and the calls that capture refuses. Every expected value is an eager
call of the same product, which the parity tests pin against the oracle."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture
def fresh():
    """A context of its own: its workspace starts empty whatever earlier tests ran."""
    c = rocm.Context(0)
    yield c
    c.close()


def _weight(ctx, n, k, seed):
    rng = np.random.default_rng(seed)
    return ctx.quantize(dev((rng.standard_normal((n, k)) * 0.02).astype(np.float32)), rocm.F32, n, k, 4, 64)


def _eager(torch, ctx, w, x, m, n):
    y = empty((m, n), torch.float32)
    ctx.linear(w, dev(x), rocm.F32, m, y, rocm.W4A8)
    return host(ctx, y).copy()


def test_captured_products_replay_nan_then_clean(ctx, oracle):
    """W4A8 at M=40, the pair and the fused MLP recorded in one graph: a replay
    with a NaN activation gives NaN outputs (int8.rs:170-173), the next replay
    with a clean one gives the eager bits again; eager products between the
    replays (crossing the flag ring twice) stay clean."""
    torch = pytest.importorskip("torch")
    m, n, k, ff = 40, 128, 256, 192
    w, w2 = _weight(ctx, n, k, 31), _weight(ctx, n, k, 32)
    gate, up = _weight(ctx, ff, k, 33), _weight(ctx, ff, k, 34)
    rng = np.random.default_rng(35)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bad = x.copy()
    bad[7, 3] = np.nan
    want = _eager(torch, ctx, w, x, m, n)
    want2 = _eager(torch, ctx, w2, x, m, n)
    q_want, s_want = empty((m, ff), torch.int8), empty((m, ff // 64), torch.float32)
    ctx.mlp_requant(gate, up, dev(x), m, q_want, s_want)
    q_want, s_want = host(ctx, q_want).copy(), host(ctx, s_want).copy()
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            xin = torch.from_numpy(x).cuda()
            y, ya, yb = (torch.empty((m, n), device="cuda") for _ in range(3))
            q, s = torch.empty((m, ff), dtype=torch.int8, device="cuda"), torch.empty((m, ff // 64), device="cuda")
            xclean, yclean = torch.from_numpy(x).cuda(), torch.empty((m, n), device="cuda")

            def record():
                ctx.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
                ctx.linear_pair(w, w2, xin, m, ya, yb, rocm.W4A8)
                ctx.mlp_requant(gate, up, xin, m, q, s)

            record()  # sizes the workspace before capture
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with rocm.capture(graph, stream):
                record()
            for i, src in enumerate([bad, x, x, bad, bad, x]):
                xin.copy_(torch.from_numpy(src))
                y.fill_(3.0)
                graph.replay()
                for _ in range(70 if i == 2 else 5):
                    ctx.linear(w, xclean, rocm.F32, m, yclean, rocm.W4A8)
                assert bits_equal(host(ctx, yclean), want), i
                got, got_a, got_b = host(ctx, y), host(ctx, ya), host(ctx, yb)
                got_q, got_s = host(ctx, q), host(ctx, s)
                if src is bad:
                    assert np.isnan(got).all() and np.isnan(got_a).all() and np.isnan(got_b).all(), i
                    assert np.isnan(got_s).all() and not got_q.any(), i
                else:
                    assert bits_equal(got, want) and bits_equal(got_a, want) and bits_equal(got_b, want2), i
                    assert bits_equal(got_q, q_want) and bits_equal(got_s, s_want), i
    finally:
        ctx.set_stream(None)
    for t in (w, w2, gate, up):
        t.free()


def test_workspace_a_graph_uses_outlives_growth(fresh, oracle):
    """A product recorded at M=40 keeps its workspace when a later eager call
    grows the context workspace: replays after the growth still give the
    eager bits."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 128, 256
    w = _weight(fresh, n, k, 41)
    x = np.random.default_rng(42).standard_normal((m, k)).astype(np.float32)
    want = _eager(torch, fresh, w, x, m, n)
    stream = torch.cuda.Stream()
    fresh.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            xin, y = torch.from_numpy(x).cuda(), torch.empty((m, n), device="cuda")
            fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with rocm.capture(graph, stream):
                fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
            # an eager product that replaces the 1 MiB first workspace
            big_m, big_k = 2048, 1024
            wb = _weight(fresh, 64, big_k, 43)
            xb = torch.randn((big_m, big_k), device="cuda")
            yb = torch.empty((big_m, 64), device="cuda")
            fresh.linear(wb, xb, rocm.F32, big_m, yb, rocm.W4A8)
            for _ in range(3):
                y.fill_(-1.0)
                graph.replay()
                assert bits_equal(host(fresh, y), want)
            wb.free()
    finally:
        fresh.set_stream(None)
    w.free()


def test_capture_refuses_growth_stream_changes_and_synchronous_calls(fresh, oracle):
    """Under capture the workspace cannot grow, the stream cannot change and
    synchronous entry points cannot run: each is INVALID_REQUEST, nothing is
    recorded, and the context works eagerly afterwards."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 64, 4096  # the fresh context has no workspace yet
    w = _weight(fresh, n, k, 51)
    x = torch.randn((m, k), device="cuda")
    y = torch.empty((m, n), device="cuda")
    raw = oracle.f32_to_bf16((np.random.default_rng(52).standard_normal((n, 256)) * 0.02).astype(np.float32))
    wire = oracle.pack_g64(raw, n, 256, 4)
    wire_a = oracle.pack_g64(np.ascontiguousarray(raw[:4]), 4, 256, 4)
    values = torch.randn((n, 256), device="cuda")
    model = fresh.pplx_create(rocm.PplxConfig(layers=1, hidden=256, ff=512, delta_heads=4, delta_key_heads=2,
                                              delta_head_dim=128, attn_heads=4, attn_kv_heads=2, attn_head_dim=256))
    stream = torch.cuda.Stream()
    fresh.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            torch.cuda.synchronize()
            # each call returns before enqueueing anything (the weight upload used to record its memsets first)
            for call in (lambda: fresh.linear(w, x, rocm.F32, m, y, rocm.W4A8),
                         lambda: fresh.set_stream(None),
                         lambda: fresh.project(w, x, 1, y),
                         lambda: fresh.sync(),
                         lambda: fresh.upload(wire, rocm.Q4_G64_F32, n, 256),
                         lambda: fresh.quantize(values, rocm.F32, n, 256, 4, 64),
                         lambda: model.set_weight("language_model.layers.0.linear_attn.in_proj_a.weight", wire_a,
                                                  rocm.Q4_G64_F32, 4, 256)):
                graph = torch.cuda.CUDAGraph()
                with pytest.raises(rocm.DzError) as e:
                    with rocm.capture(graph, stream):
                        y.zero_()
                        call()
                assert e.value.code == "INVALID_REQUEST"
            fresh.linear(w, x, rocm.F32, m, y, rocm.W4A8)
            got = host(fresh, y)
            fresh.upload(wire, rocm.Q4_G64_F32, n, 256).free()  # eager again: fine
    finally:
        fresh.set_stream(None)
        model.close()
    xs = x[:40].cpu().numpy()
    assert bits_equal(got[:40], _eager(torch, fresh, w, xs, 40, n))
    w.free()


def test_stream_change_waits_for_products_on_the_old_stream(ctx, oracle):
    """Products queued on one stream, then more on another after dz_set_stream:
    the second stream's flag-ring clear cannot overtake the first stream's
    products, so the NaN call is NaN and every other call keeps the eager bits."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 512, 4096
    w = _weight(ctx, n, k, 61)
    rng = np.random.default_rng(62)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bad = x.copy()
    bad[0, 0] = np.inf
    want = _eager(torch, ctx, w, x, m, n)
    xd, bd = dev(x), dev(bad)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ys = [empty((m, n), torch.float32) for _ in range(120)]
    try:
        ctx.set_stream(s1.cuda_stream)
        for i in range(60):
            ctx.linear(w, bd if i == 59 else xd, rocm.F32, m, ys[i], rocm.W4A8)
        ctx.set_stream(s2.cuda_stream)
        for i in range(60, 120):
            ctx.linear(w, xd, rocm.F32, m, ys[i], rocm.W4A8)
        ctx.sync()
    finally:
        ctx.set_stream(None)
    torch.cuda.synchronize()
    for i, y in enumerate(ys):
        got = y.cpu().numpy()
        if i == 59:
            assert np.isnan(got).all()
        else:
            assert bits_equal(got, want), i
    w.free()


def test_capture_release_gives_flag_slots_back(fresh, oracle):
    """45 graphs of 100 recorded W4A8 products at M=40 (4,500 recordings, more
    than the 4,032 flag slots), each destroyed and released before the next:
    every recording succeeds and every replay keeps the eager bits, NaN replays
    stay NaN on reused slots, and the context reports no held slot at the end.
    Two graphs kept at once are given back by dz_capture_release_all. The
    current capture cannot be released while it records, and dz_capture_id
    outside a capture is INVALID_REQUEST."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 64, 256
    w = _weight(fresh, n, k, 71)
    rng = np.random.default_rng(72)
    x = rng.standard_normal((m, k)).astype(np.float32)
    bad = x.copy()
    bad[5, 9] = np.nan
    want = _eager(torch, fresh, w, x, m, n)
    with pytest.raises(rocm.DzError) as e:
        fresh.capture_id()
    assert e.value.code == "INVALID_REQUEST"
    stream = torch.cuda.Stream()
    fresh.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            xin, y = torch.from_numpy(x).cuda(), torch.empty((m, n), device="cuda")
            fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)  # sizes the workspace
            torch.cuda.synchronize()
            for rep in range(45):
                graph = torch.cuda.CUDAGraph()
                with rocm.capture(graph, stream):
                    cid = fresh.capture_id()
                    for _ in range(100):
                        fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
                    if rep == 0:
                        for call in (lambda: fresh.capture_release(cid), fresh.capture_release_all):
                            with pytest.raises(rocm.DzError) as e:
                                call()
                            assert e.value.code == "INVALID_REQUEST"
                slots = fresh.info()["capture_slots"]
                assert slots["held"] == 100 and slots["captures"] == 1, (rep, slots)
                for src in ([bad, x] if rep % 10 == 9 else [x]):
                    xin.copy_(torch.from_numpy(src))
                    y.fill_(2.0)
                    graph.replay()
                    got = host(fresh, y)
                    if src is bad:
                        assert np.isnan(got).all(), rep
                    else:
                        assert bits_equal(got, want), rep
                torch.cuda.synchronize()
                graph.reset()
                fresh.capture_release(cid)
                assert fresh.info()["capture_slots"]["held"] == 0, rep
            graphs = []
            for _ in range(2):
                graph = torch.cuda.CUDAGraph()
                with rocm.capture(graph, stream):
                    for _ in range(100):
                        fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
                graphs.append(graph)
            slots = fresh.info()["capture_slots"]
            assert slots["held"] == 200 and slots["captures"] == 2, slots
            for graph in graphs:
                y.fill_(2.0)
                graph.replay()
                assert bits_equal(host(fresh, y), want)
            torch.cuda.synchronize()
            for graph in graphs:
                graph.reset()
            fresh.capture_release_all()
            assert fresh.info()["capture_slots"]["held"] == 0
            assert fresh.info()["capture_slots"]["captures"] == 0
    finally:
        fresh.set_stream(None)
    w.free()


def test_capture_release_frees_the_retired_workspace(fresh, oracle):
    """A graph recorded at M=40 keeps its workspace alive when an eager call
    grows the context workspace (one retired workspace); once the graph is
    destroyed and its capture released, the retired workspace is freed, and a
    new recording on the grown workspace keeps the eager bits."""
    torch = pytest.importorskip("torch")
    m, n, k = 40, 128, 256
    w = _weight(fresh, n, k, 81)
    x = np.random.default_rng(82).standard_normal((m, k)).astype(np.float32)
    want = _eager(torch, fresh, w, x, m, n)
    stream = torch.cuda.Stream()
    fresh.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.stream(stream):
            xin, y = torch.from_numpy(x).cuda(), torch.empty((m, n), device="cuda")
            fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with rocm.capture(graph, stream):
                cid = fresh.capture_id()
                fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
            big_m, big_k = 2048, 1024
            wb = _weight(fresh, 64, big_k, 83)
            xb = torch.randn((big_m, big_k), device="cuda")
            yb = torch.empty((big_m, 64), device="cuda")
            fresh.linear(wb, xb, rocm.F32, big_m, yb, rocm.W4A8)
            assert fresh.info()["capture_slots"]["retired_workspaces"] == 1
            y.fill_(-1.0)
            graph.replay()
            assert bits_equal(host(fresh, y), want)
            torch.cuda.synchronize()
            graph.reset()
            fresh.capture_release(cid)
            assert fresh.info()["capture_slots"]["retired_workspaces"] == 0
            graph = torch.cuda.CUDAGraph()
            with rocm.capture(graph, stream):
                fresh.linear(w, xin, rocm.F32, m, y, rocm.W4A8)
            for _ in range(2):
                y.fill_(-1.0)
                graph.replay()
                assert bits_equal(host(fresh, y), want)
            wb.free()
    finally:
        fresh.set_stream(None)
    w.free()
