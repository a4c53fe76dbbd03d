"""gsdh_gqa_attention_noalloc (split partials in the library's static device
scratch, no allocation in the call) against gsdh_gqa_attention on the same
inputs, through the C ABI: two calls in a row, the second smaller, then a
size beyond the scratch rejected on the host.  Then both entry points under
HIP graph capture: one captured call replayed three times with q and a cache
row changed between the replays (and a call of another shape in between),
every replay against the oracle; a stream with a workspace of its own; and a
merge whose bounded wait runs out (forced from the host: the merging blocks
wait for a tag no split writes) reported by gsdh_stream_sync."""
import ctypes
import os

import numpy as np
import pytest

import oracle as O
from conftest import rel_l2
from gpu_util import D, E, H, banner, p

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    from gsdlq import hip
    name, total, ncu = hip.device_info()     # raises when no GPU is visible
    assert ncu > 0, name
    return hip.lib()


def _inputs(ctx, nh, nkv, hd, seed):
    from gsdlq import pack
    ms = ctx + 3
    kc = pack.synth_f16(seed, ctx, ms * nkv * hd, 1.0)
    vc = pack.synth_f16(seed + 1, ctx, ms * nkv * hd, 1.0)
    q = np.random.default_rng(seed).standard_normal(nh * hd).astype(np.float32)
    return ms, q, kc, vc


def _run(lib, fn, ctx, nh, nkv, hd, ms, dq, dk, dv):
    out = E(nh * hd * 4)
    getattr(lib, fn)(None, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms, 1.0 / float(np.sqrt(hd)))
    return H(out, np.float32, nh * hd)


def _oracle(q, kc, vc, ctx, nh, nkv, hd, ms):
    ref = np.zeros(nh * hd, np.float32)
    O.load("port").gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(ref), 0, ctx - 1, nh, nkv, hd, ms,
                                         1.0 / float(np.sqrt(hd)))
    return ref


def test_noalloc_attention_matches_allocating_entry(lib):
    # 8192 positions (32 splits of 8 KV heads), then a smaller call: 2000
    # positions of 4 KV heads (fewer splits, another word layout)
    for ctx, nh, nkv, hd, seed in [(8192, 32, 8, 128, 71), (2000, 16, 4, 128, 72)]:
        banner(f"no-alloc attention ctx {ctx} heads {nh}/{nkv} hd {hd}")
        ms, q, kc, vc = _inputs(ctx, nh, nkv, hd, seed)
        dq, dk, dv = D(q), D(kc), D(vc)
        want = _run(lib, "gsdh_gqa_attention", ctx, nh, nkv, hd, ms, dq, dk, dv)
        got = _run(lib, "gsdh_gqa_attention_noalloc", ctx, nh, nkv, hd, ms, dq, dk, dv)
        assert rel_l2(got, want) < 1e-3
        assert np.array_equal(got, want)   # the same kernel and split plan
        assert rel_l2(got, _oracle(q, kc, vc, ctx, nh, nkv, hd, ms)) < 1e-3


def test_noalloc_attention_rejects_oversize(lib):
    from gsdlq.hip import HipError
    y = E(64)
    # 64 KV heads x 8 query heads each x 256 dims at 65536 positions: far
    # beyond 8 MiB of partials (rejected before any launch)
    with pytest.raises(HipError, match="static scratch"):
        lib.gsdh_gqa_attention_noalloc(None, p(y), p(y), p(y), p(y), 0, 65535, 512, 64, 256, 65536, 0.0625)


def _h2d(lib, dst, offset, arr, stream):
    a = np.ascontiguousarray(arr)
    lib.gsdh_memcpy_h2d(ctypes.c_void_p(dst.ptr.value + offset), a.ctypes.data_as(ctypes.c_void_p), a.nbytes, stream)


def _d2h(lib, src, count, stream):
    out = np.empty(count, np.float32)
    lib.gsdh_memcpy_d2h(out.ctypes.data_as(ctypes.c_void_p), src.ptr, count * 4, stream)
    lib.gsdh_stream_sync(stream)
    return out


def _graph_replays(lib, fn, ctx, nh, nkv, hd, seed, workspace=False, warm=True):
    """One call of `fn` captured on a stream of its own, replayed three times;
    before each replay a new q and a new cache row (position ctx // 2), and
    an eager call of another shape on the same stream (its words in the same
    memory); every replay against the oracle on the replay's inputs."""
    from gsdlq import pack
    ms, q, kc, vc = _inputs(ctx, nh, nkv, hd, seed)
    sc = 1.0 / float(np.sqrt(hd))
    st = ctypes.c_void_p()
    lib.gsdh_stream_create(ctypes.byref(st))
    ge = ctypes.c_void_p()
    try:
        if workspace:
            lib.gsdh_attention_workspace_create(st, nkv, nh, hd, ms)
        dq, dk, dv, out = D(q), D(kc), D(vc), E(nh * hd * 4)
        # the other shape: 4 KV heads x 2, head dim 64, 3000 positions
        oms, oq, okc, ovc = _inputs(3000, 8, 4, 64, seed + 7)
        odq, odk, odv, oout = D(oq), D(okc), D(ovc), E(8 * 64 * 4)
        oref = _oracle(oq, okc, ovc, 3000, 8, 4, 64, oms)
        if warm:   # an eager call first (the allocating twin's old first-call path)
            getattr(lib, fn)(st, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms, sc)
            lib.gsdh_stream_sync(st)
            assert rel_l2(_d2h(lib, out, nh * hd, st), _oracle(q, kc, vc, ctx, nh, nkv, hd, ms)) < 1e-3
        lib.gsdh_stream_begin_capture(st)
        getattr(lib, fn)(st, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms, sc)
        lib.gsdh_stream_end_capture(st, ctypes.byref(ge))
        rng = np.random.default_rng(seed + 100)
        row = ctx // 2
        for rep in range(3):
            banner(f"{fn} graph replay {rep} ctx {ctx} heads {nh}/{nkv} hd {hd} workspace {workspace}")
            q = rng.standard_normal(nh * hd).astype(np.float32)
            krow = pack.synth_f16(seed + 200 + rep, 0, nkv * hd, 1.0)
            vrow = pack.synth_f16(seed + 300 + rep, 0, nkv * hd, 1.0)
            kc[row * nkv * hd:(row + 1) * nkv * hd] = krow
            vc[row * nkv * hd:(row + 1) * nkv * hd] = vrow
            _h2d(lib, dq, 0, q, st)
            _h2d(lib, dk, row * nkv * hd * 2, krow, st)
            _h2d(lib, dv, row * nkv * hd * 2, vrow, st)
            getattr(lib, fn)(st, p(odq), p(odk), p(odv), p(oout), 0, 2999, 8, 4, 64, oms, 0.125)
            lib.gsdh_graph_replay(ge, st)
            lib.gsdh_stream_sync(st)
            got = _d2h(lib, out, nh * hd, st)
            assert rel_l2(got, _oracle(q, kc, vc, ctx, nh, nkv, hd, ms)) < 1e-3, (fn, ctx, rep)
            assert rel_l2(_d2h(lib, oout, 8 * 64, st), oref) < 1e-3, (fn, ctx, rep, "other shape")
    finally:
        if ge.value:
            lib.gsdh_graph_destroy(ge)
        lib.gsdh_stream_destroy(st)


@pytest.mark.parametrize("ctx", [2048, 8192])
def test_noalloc_attention_graph_replays(lib, ctx):
    # 8 KV heads x 32 splits: 256 blocks, eight merging blocks per KV head
    # that wait on blocks dispatched after their own
    _graph_replays(lib, "gsdh_gqa_attention_noalloc", ctx, 32, 8, 128, seed=80 + ctx % 7, warm=False)


@pytest.mark.parametrize("ctx,workspace", [(2048, False), (8192, False), (2048, True)])
def test_attention_graph_replays_after_warmup(lib, ctx, workspace):
    _graph_replays(lib, "gsdh_gqa_attention", ctx, 32, 8, 128, seed=90 + ctx % 11, workspace=workspace)


def test_attention_workspace_too_small_rejected(lib):
    from gsdlq.hip import HipError
    st = ctypes.c_void_p()
    lib.gsdh_stream_create(ctypes.byref(st))
    try:
        assert lib.gsdh_attention_workspace_bytes(8, 32, 128, 1024) > 256
        lib.gsdh_attention_workspace_create(st, 8, 32, 128, 1024)
        y = E(64)
        with pytest.raises(HipError, match="stream's workspace"):
            lib.gsdh_gqa_attention(st, p(y), p(y), p(y), p(y), 0, 8191, 32, 8, 128, 8192, 0.088)
    finally:
        lib.gsdh_stream_destroy(st)


def test_attention_wait_timeout_reported(lib):
    """The merging blocks wait for a tag no split writes (a test setting of
    the host), so every merge gives up after 64 polling rounds and sets the
    error word; the next synchronisation reports it.  Then an ordinary call
    on the same scratch is correct and reports nothing."""
    from gsdlq.hip import HipError
    ctx, nh, nkv, hd = 2048, 32, 8, 128
    ms, q, kc, vc = _inputs(ctx, nh, nkv, hd, 61)
    dq, dk, dv, out = D(q), D(kc), D(vc), E(nh * hd * 4)
    os.environ["GSD_ATTN_TEST_SKEW"] = "1"
    os.environ["GSD_ATTN_SPIN_LIMIT"] = "64"
    try:
        banner("attention: forced merge timeout")
        lib.gsdh_gqa_attention_noalloc(None, p(dq), p(dk), p(dv), p(out), 0, ctx - 1, nh, nkv, hd, ms,
                                       1.0 / float(np.sqrt(hd)))
        with pytest.raises(HipError, match="timed out"):
            lib.gsdh_stream_sync(None)
    finally:
        del os.environ["GSD_ATTN_TEST_SKEW"]
        del os.environ["GSD_ATTN_SPIN_LIMIT"]
    lib.gsdh_stream_sync(None)   # reported once, then clear
    got = _run(lib, "gsdh_gqa_attention_noalloc", ctx, nh, nkv, hd, ms, dq, dk, dv)
    assert rel_l2(got, _oracle(q, kc, vc, ctx, nh, nkv, hd, ms)) < 1e-3
