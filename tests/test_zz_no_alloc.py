"""dz_linear_noalloc: the entry point that allocates nothing. Its results are
compared bit for bit with dz_linear's (which the product tests pin against the
oracle), over consecutive calls whose second input is smaller, a NaN call
followed by a clean one, its size limit and a graph recorded on a context that
has no workspace at all."""
import numpy as np
import pytest

from decisive_amd import rocm
from tests.gpu_util import bits_equal, dev, empty, host

pytestmark = pytest.mark.gpu


def _weight(ctx, oracle, n, k, bits, seed):
    rng = np.random.default_rng(seed)
    raw = oracle.f32_to_bf16((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    return raw, ctx.quantize(dev(raw), rocm.BF16, n, k, bits, 64)


def _both(torch, ctx, w, x, m, n, mode, x_dtype=rocm.F32):
    xd = dev(x)
    a, b = empty((m, n), torch.float32), empty((m, n), torch.float32)
    ctx.linear(w, xd, x_dtype, m, a, mode)
    ctx.linear_noalloc(w, xd, x_dtype, m, b, mode)
    return host(ctx, a), host(ctx, b)


@pytest.mark.parametrize("wb,ab", [(4, 8), (8, 8), (4, 4)])
def test_noalloc_equals_linear_on_two_calls_the_second_smaller(ctx, oracle, wb, ab):
    torch = pytest.importorskip("torch")
    n, k = 520, 4096
    raw, w = _weight(ctx, oracle, n, k, wb, 71 + wb + ab)
    rng = np.random.default_rng(72)
    mode = rocm.W4A4 if ab == 4 else rocm.W4A8
    codes, scales = oracle.weight_quantize(raw, n, k, wb)
    for m in (300, 40):
        x = (rng.standard_normal((m, k)) * 1.5).astype(np.float32)
        want, got = _both(torch, ctx, w, x, m, n, mode)
        assert bits_equal(got, want), m
        assert bits_equal(got, oracle.matrix_apply(x, m, codes, scales, n, k, ab, fused=True)), m
    w.free()


def test_noalloc_nan_call_then_clean_smaller_call(ctx, oracle):
    """The scratch keeps the last call's contents: the flag is cleared by each
    call, so a NaN activation makes only its own call NaN."""
    torch = pytest.importorskip("torch")
    n, k = 200, 1088
    _, w = _weight(ctx, oracle, n, k, 4, 73)
    rng = np.random.default_rng(74)
    x = rng.standard_normal((257, k)).astype(np.float32)
    x[100, 9] = np.nan
    y = empty((257, n), torch.float32)
    ctx.linear_noalloc(w, dev(x), rocm.F32, 257, y, rocm.W4A8)
    assert np.isnan(host(ctx, y)).all()
    x2 = rng.standard_normal((33, k)).astype(np.float32)
    want, got = _both(torch, ctx, w, x2, 33, n, rocm.W4A8)
    assert not np.isnan(got).any() and bits_equal(got, want)
    w.free()


@pytest.mark.parametrize("m", [1, 9, 16])
def test_noalloc_few_rows_and_w4a16_pass_through(ctx, oracle, m):
    torch = pytest.importorskip("torch")
    n, k = 96, 512
    _, w = _weight(ctx, oracle, n, k, 4, 75)
    x = np.random.default_rng(76 + m).standard_normal((m, k)).astype(np.float32)
    want, got = _both(torch, ctx, w, x, m, n, rocm.W4A8)
    assert bits_equal(got, want)
    wf = (np.random.default_rng(77).standard_normal((n, k)) * 0.02).astype(np.float32)
    w16 = ctx.quantize(dev(wf), rocm.F32, n, k, 4, 32)
    for rows in (m, 40):
        xh = np.random.default_rng(78 + rows).standard_normal((rows, k)).astype(np.float16)
        want, got = _both(torch, ctx, w16, xh, rows, n, rocm.W4A16, rocm.F16)
        assert bits_equal(got, want), rows
    w.free()
    w16.free()


def test_noalloc_size_limit(ctx, oracle):
    """3,855 rows of 4096 columns fill the 16 MiB scratch; one more row is
    RESOURCE_LIMIT and launches nothing."""
    torch = pytest.importorskip("torch")
    n, k = 64, 4096
    _, w = _weight(ctx, oracle, n, k, 4, 79)
    x = torch.randn((3856, k), device="cuda")
    a, b = empty((3856, n), torch.float32), empty((3856, n), torch.float32)
    ctx.linear(w, x, rocm.F32, 3855, a, rocm.W4A8)
    ctx.linear_noalloc(w, x, rocm.F32, 3855, b, rocm.W4A8)
    assert bits_equal(host(ctx, b)[:3855], host(ctx, a)[:3855])
    b.fill_(5.0)
    with pytest.raises(rocm.DzError) as e:
        ctx.linear_noalloc(w, x, rocm.F32, 3856, b, rocm.W4A8)
    assert e.value.code == "RESOURCE_LIMIT"
    assert (host(ctx, b) == 5.0).all()
    w.free()


def test_noalloc_records_on_a_context_without_workspace(oracle):
    """A fresh context has no workspace, so dz_linear cannot be recorded at
    m > 16 before an eager call; dz_linear_noalloc can, and every replay equals
    the eager dz_linear result, including after a NaN replay."""
    torch = pytest.importorskip("torch")
    fresh = rocm.Context(0)
    try:
        n, k, m = 128, 640, 48
        raw, w = _weight(fresh, oracle, n, k, 4, 80)
        rng = np.random.default_rng(81)
        x = rng.standard_normal((m, k)).astype(np.float32)
        bad = x.copy()
        bad[0, 1] = -np.inf
        codes, scales = oracle.weight_quantize(raw, n, k, 4)
        want = oracle.matrix_apply(x, m, codes, scales, n, k, 8, fused=True)
        stream = torch.cuda.Stream()
        fresh.set_stream(stream.cuda_stream)
        try:
            with torch.cuda.stream(stream):
                xin, y = torch.from_numpy(x).cuda(), torch.empty((m, n), device="cuda")
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with rocm.capture(graph, stream):
                    fresh.linear_noalloc(w, xin, rocm.F32, m, y, rocm.W4A8)
                for src in (x, bad, x, x):
                    xin.copy_(torch.from_numpy(src))
                    y.fill_(2.0)
                    graph.replay()
                    got = host(fresh, y)
                    if src is bad:
                        assert np.isnan(got).all()
                    else:
                        assert bits_equal(got, want)
                    # eager use of the same scratch between replays
                    y2 = torch.empty((40, n), device="cuda")
                    fresh.linear_noalloc(w, xin[:40], rocm.F32, 40, y2, rocm.W4A8)
                    fresh.sync()
        finally:
            fresh.set_stream(None)
        w.free()
    finally:
        fresh.close()
