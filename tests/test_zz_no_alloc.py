"""faq_attention_fwd_split_noalloc: the split-key attention on the library's static per-GPU
scratch array, against faq_attention_fwd_split with a caller workspace (same kernels, same
split count: bitwise equal outputs and denominators), twice in a row with the second call
smaller, and its refusal of a call whose layout exceeds the array.  Called through the C
ABI (ctypes)."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _operands(dev, seed, B, Hq, Hkv, Lq, Lk):
    from faquant_amd import _ops

    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, Hq, Lq, 128, generator=g).to(dev, torch.bfloat16)
    k = torch.randn(B, Hkv, Lk, 128, generator=g).to(dev, torch.bfloat16)
    v = torch.randn(B, Hkv, Lk, 128, generator=g).to(dev, torch.bfloat16)
    qh, _ = _ops.operand_prep(q, levels="123")
    kh, _ = _ops.operand_prep(k, levels="123")
    vt = _ops.operand_prep_vt(v, levels="123")
    return qh, kh, vt


def _call(lib, dev, qh, kh, vt, Lk, nsplit, *, noalloc):
    from faquant_amd import _lib

    B, Hq, Lq, _ = qh.shape
    Hkv = kh.shape[1]
    out = torch.full((B, Hq, Lq, 128), float("nan"), device=dev, dtype=torch.float32)
    den = torch.full((B, Hq, Lq), float("nan"), device=dev, dtype=torch.float32)
    common = (
        qh.data_ptr(), *qh.stride()[:3], kh.data_ptr(), *kh.stride()[:3], vt.data_ptr(), *vt.stride()[:3],
        vt.shape[-1], out.data_ptr(), _lib.F32, *out.stride()[:3],
        B, Hq, Hkv, Lq, Lk, 1, 128**-0.5, 1, 123, 1, den.data_ptr(), nsplit,
    )
    stream = _lib.stream_ptr(dev)
    if noalloc:
        rc = lib.faq_attention_fwd_split_noalloc(*common, None, stream)
    else:
        ws_bytes = lib.faq_attention_split_workspace(B, Hq, Lq, Lk, nsplit)
        ws = torch.empty(int(ws_bytes), device=dev, dtype=torch.uint8)
        rc = lib.faq_attention_fwd_split(*common, ws.data_ptr(), ws.numel(), None, stream)
    return rc, out, den


def test_noalloc_split_equals_workspace_split(dev):
    from faquant_amd import _lib

    lib = _lib.load()
    # a decode step of Qwen3-8B at 32k keys, then a smaller one (fewer heads, keys and ranges)
    for (B, Hq, Hkv, Lq, Lk, nsplit) in ((1, 32, 8, 1, 32768, 32), (1, 8, 2, 3, 3000, 5)):
        print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} Lq={Lq} Lk={Lk} nsplit={nsplit}", flush=True)
        qh, kh, vt = _operands(dev, Lk, B, Hq, Hkv, Lq, Lk)
        rc_a, out_a, den_a = _call(lib, dev, qh, kh, vt, Lk, nsplit, noalloc=False)
        rc_b, out_b, den_b = _call(lib, dev, qh, kh, vt, Lk, nsplit, noalloc=True)
        torch.cuda.synchronize()
        assert rc_a == _lib.OK and rc_b == _lib.OK, lib.faq_last_error()
        assert torch.isfinite(out_b).all()
        assert torch.equal(out_a, out_b)
        assert torch.equal(den_a, den_b)


def test_noalloc_refuses_a_layout_beyond_the_array(dev):
    from faquant_amd import _lib

    lib = _lib.load()
    B, Hq, Lq, Lk, nsplit = 4, 64, 64, 65536, 64
    need = lib.faq_attention_split_workspace(B, Hq, Lq, Lk, nsplit)
    assert need > 8 << 20
    qh, kh, vt = _operands(dev, 1, 1, 2, 1, 1, 256)
    rc, _, _ = _call(lib, dev, qh, kh, vt, 256, 1, noalloc=True)
    assert rc == _lib.OK
    rc = lib.faq_attention_fwd_split_noalloc(
        qh.data_ptr(), 0, 0, 128, kh.data_ptr(), 0, 0, 128, vt.data_ptr(), 0, 0, 65536, 65536,
        qh.data_ptr(), _lib.F32, 0, 0, 128, B, Hq, 8, Lq, Lk, 1, 0.1, 1, 123, 1, None, nsplit, None,
        _lib.stream_ptr(dev))
    assert rc == _lib.EINVAL
    assert "static buffer" in lib.faq_last_error().decode()
    np.testing.assert_equal(int(need) > 0, True)
