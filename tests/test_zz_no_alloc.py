"""The no-allocation attention entry point against the allocating one.

vh_flash_attention_f32_da3_base_into keeps its key-split partials in the
library's per-GPU scratch array and writes a caller-provided output; it must
give the same bits as vh_flash_attention_f32_da3_base, call after call (the
second call here is smaller, so stale partials of the first would show), and
reject shapes past its scratch before launching anything.
"""
import numpy as np
import pytest

import vestra_hip as vh
from conftest import assert_bits_equal
from vestra_hip import seeded

pytestmark = pytest.mark.gpu

MAX_ROWS = 63550  # heads*tokens whose 4-way key-split partials fit 64 MiB


def _qkv(rt, heads, tokens, seed):
    n = heads * tokens * 64
    return [rt.upload_f32(seeded.normal(seed + i, n)) for i in range(3)]


@pytest.mark.parametrize("token_major", [True, False])
def test_no_alloc_attention_matches_allocating_entry(rt, token_major):
    # 12 x 865 splits the keys three ways; 5 x 300 and 2 x 64 are smaller.
    for heads, tokens, seed in ((12, 865, 10), (5, 300, 20), (2, 64, 30)):
        q, k, v = _qkv(rt, heads, tokens, seed)
        exp = rt.download_f32(rt.flash_attention_f32_da3_base(q, k, v, heads, tokens, token_major))
        out = rt.alloc_f32(heads * tokens * 64)
        rt.flash_attention_f32_da3_base_into(q, k, v, heads, tokens, token_major, out)
        got = rt.download_f32(out)
        assert np.isfinite(got).all()
        assert_bits_equal(got, exp, f"no-alloc attention {heads}x{tokens}")


def test_no_alloc_attention_rejects_before_launch(rt):
    heads, tokens = 1, MAX_ROWS + 1
    q, k, v = _qkv(rt, heads, tokens, 40)
    fill = np.full(heads * tokens * 64, 7.0, np.float32)
    out = rt.upload_f32(fill)
    with pytest.raises(vh.KernelError, match="no-allocation limit"):
        rt.flash_attention_f32_da3_base_into(q, k, v, heads, tokens, True, out)
    with pytest.raises(vh.LengthMismatch):
        rt.flash_attention_f32_da3_base_into(q, k, v, heads, tokens - 1, True, out)
    assert np.array_equal(rt.download_f32(out), fill)
    # the largest accepted shape still runs and matches
    q, k, v = (rt.upload_f32(np.asarray(rt.download_f32(t))[:MAX_ROWS * 64]) for t in (q, k, v))
    out = rt.alloc_f32(MAX_ROWS * 64)
    rt.flash_attention_f32_da3_base_into(q, k, v, 1, MAX_ROWS, False, out)
    exp = rt.download_f32(rt.flash_attention_f32_da3_base(q, k, v, 1, MAX_ROWS, False))
    assert_bits_equal(rt.download_f32(out), exp, "no-alloc attention at the limit")


def test_no_alloc_attention_two_runtimes_back_to_back(rt):
    """Two runtimes (two streams) share the GPU's scratch array: each call
    waits for the previous call's launch, so back-to-back calls without a
    host synchronisation between them give the allocating entry point's bits
    (12 x 865 and 8 x 865 both split the keys across workgroups, so both
    launches write partials)."""
    other = vh.Runtime(0)
    cases = ((rt, 12, 865, 50), (other, 8, 865, 60), (rt, 12, 865, 70), (other, 3, 600, 80))
    inputs, outs, exps = [], [], []
    for r, heads, tokens, seed in cases:
        q, k, v = _qkv(r, heads, tokens, seed)
        inputs.append((q, k, v))
        exps.append(r.download_f32(r.flash_attention_f32_da3_base(q, k, v, heads, tokens, True)))
        outs.append(r.alloc_f32(heads * tokens * 64))
    rt.synchronize()
    other.synchronize()
    for (r, heads, tokens, _), (q, k, v), out in zip(cases, inputs, outs):
        r.flash_attention_f32_da3_base_into(q, k, v, heads, tokens, True, out)
    for (r, heads, tokens, _), out, exp in zip(cases, outs, exps):
        assert_bits_equal(r.download_f32(out), exp, f"no-alloc attention {heads}x{tokens} on two streams")
