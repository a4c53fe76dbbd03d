"""gsdh_gqa_attention_noalloc (split partials in the library's static device
scratch, no allocation in the call) against gsdh_gqa_attention on the same
inputs, through the C ABI: two calls in a row, the second smaller, then a
size beyond the scratch rejected on the host."""
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
        ref = np.zeros(nh * hd, np.float32)
        O.load("port").gsd_cpu_gqa_attention(O.P(q), O.P(kc), O.P(vc), O.P(ref), 0, ctx - 1, nh, nkv, hd, ms,
                                             1.0 / float(np.sqrt(hd)))
        assert rel_l2(got, ref) < 1e-3


def test_noalloc_attention_rejects_oversize(lib):
    from gsdlq.hip import HipError
    y = E(64)
    # 64 KV heads x 8 query heads each x 256 dims at 65536 positions: far
    # beyond 8 MiB of partials (rejected before any launch)
    with pytest.raises(HipError, match="static scratch"):
        lib.gsdh_gqa_attention_noalloc(None, p(y), p(y), p(y), p(y), 0, 65535, 512, 64, 256, 65536, 0.0625)
