"""Work-item streaming in the attention kernel.

One workgroup per CU runs its work items one after another: rounds of items, every second
round in reverse inside each XCD's share, and the DMA of the next item's first key tile
issued during the current item's last tile.  A row's result must not depend on which
workgroup, round or stream position computes it.  Each case launches many more items
than the GPU has CUs, then recomputes the rows in launches small enough for one item per
workgroup (one batch element, or a subset of heads) and requires bitwise equality.  The
masked cases put empty items (fully padded batch rows, or rows whose window holds no key)
between full ones, which exercises the cross-item prefetch around items without tiles.
Parity with the oracle for these schedules is covered by the full-size sampled-row tests
(test_gpu_attention.py).
"""

from __future__ import annotations

import pytest

from faquant_amd import _ops

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _operands(seed, B, Hq, Hkv, L, dev, levels="123"):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, Hq, L, 128, generator=g).mul(2).to(torch.bfloat16).to(dev)
    k = torch.randn(B, Hkv, L, 128, generator=g).to(torch.bfloat16).to(dev)
    v = torch.randn(B, Hkv, L, 128, generator=g).to(torch.bfloat16).to(dev)
    qh, _ = _ops.operand_prep(q, levels=levels)
    kh, _ = _ops.operand_prep(k, levels=levels)
    vt = _ops.operand_prep_vt(v, levels=levels)
    return qh, kh, vt


def _run(qh, kh, vt, L, causal, ranges=None, out_dtype=torch.float32):
    B, Hq = qh.shape[0], qh.shape[1]
    out = torch.empty((B, L, Hq, 128), device=qh.device, dtype=out_dtype)
    den = torch.empty((B, Hq, L), device=qh.device, dtype=torch.float32)
    _ops.attention_fwd(qh, kh, vt, L, causal=causal, scale=128**-0.5, quant_p=True, p_levels=123, norm_same=True,
                       out=out.transpose(1, 2), row_den=den, ranges=ranges, split=1)
    return out, den


def _slice_ranges(r, b):
    return _ops.KeyRanges(r.row_lo[b : b + 1], r.row_hi[b : b + 1], r.row_blocks[b : b + 1], r.key_bits[b : b + 1])


def _cus(dev):
    return torch.cuda.get_device_properties(dev).multi_processor_count


@pytest.mark.parametrize("B,Hq,Hkv,L,causal", [(8, 8, 8, 2304, True), (4, 32, 8, 2048, True), (2, 24, 24, 2600, False)],
                         ids=["mha_causal", "gqa_causal", "mha_ragged_noncausal"])
def test_streamed_rows_equal_one_item_per_workgroup(dev, B, Hq, Hkv, L, causal):
    qh, kh, vt = _operands(B * 1000 + L, B, Hq, Hkv, L, dev)
    G = Hq // Hkv
    hpw = 8 if G % 8 == 0 else 4 if G % 4 == 0 else 2 if G % 2 == 0 else 1
    items = B * Hkv * (G // hpw) * -(-L // (256 // hpw))
    assert items > 2 * _cus(dev), "the case must stream at least three rounds of items"
    full, full_den = _run(qh, kh, vt, L, causal)
    for b in range(B):
        print(f"[stream] B={B} Hq={Hq} L={L} batch {b}", flush=True)
        one, one_den = _run(qh[b : b + 1], kh[b : b + 1], vt[b : b + 1], L, causal)
        assert torch.equal(one[0], full[b])
        assert torch.equal(one_den[0], full_den[b])


@pytest.mark.parametrize("window", [None, 200])
def test_streamed_rows_with_empty_items_equal_per_batch(dev, window):
    """Padding masks with fully padded batch rows: their items hold no key tile."""
    B, Hq, Hkv, L = 6, 16, 4, 1536
    qh, kh, vt = _operands(77, B, Hq, Hkv, L, dev)
    mask = torch.ones((B, L), dtype=torch.int64)
    mask[1] = 0                      # a fully padded batch row: empty items
    mask[2, : L // 3] = 0            # left padding
    mask[3, L - 100 :] = 0           # right padding
    mask[4] = 0                      # another fully padded row
    mask[5, 700:900] = 0             # a hole
    mask = mask.to(dev)
    ranges = _ops.attention_key_ranges(mask, B, L, L, causal=True, window=window)
    items = B * Hkv * -(-L // 64)
    assert items > _cus(dev)
    full, full_den = _run(qh, kh, vt, L, True, ranges)
    for b in range(B):
        print(f"[stream-mask] window={window} batch {b}", flush=True)
        one, one_den = _run(qh[b : b + 1], kh[b : b + 1], vt[b : b + 1], L, True, _slice_ranges(ranges, b))
        assert torch.equal(one[0], full[b])
        assert torch.equal(one_den[0], full_den[b])
    # fully padded rows see no key: zero output and denominator (sfa:870-884)
    assert torch.count_nonzero(full[1]) == 0 and torch.count_nonzero(full_den[4]) == 0


def test_streamed_heads_equal_head_subsets(dev):
    """Non-causal MHA (the Wan layout): all 40 heads at once versus five launches of 8."""
    B, H, L = 1, 40, 1792
    qh, kh, vt = _operands(5, B, H, H, L, dev)
    full, full_den = _run(qh, kh, vt, L, False, out_dtype=torch.bfloat16)
    for h0 in range(0, H, 8):
        part, part_den = _run(qh[:, h0 : h0 + 8].contiguous(), kh[:, h0 : h0 + 8].contiguous(),
                              vt[:, h0 : h0 + 8].contiguous(), L, False, out_dtype=torch.bfloat16)
        assert torch.equal(part, full[:, :, h0 : h0 + 8])
        assert torch.equal(part_den, full_den[:, h0 : h0 + 8])


def test_xcd_pacing_changes_no_bits(dev, monkeypatch):
    """Long non-causal items (128 key tiles and more) run with the XCD pacing counters, which
    only delay workgroups that are ahead of their XCD: the outputs and row denominators equal
    those of the same launch with pacing off (FAQ_ATTN_PACE=0), bit for bit, on consecutive
    launches (new epochs) and with more items than workgroups."""
    B, H, L = 1, 16, 16384
    qh, kh, vt = _operands(41, B, H, H, L, dev)
    print(f"[pace] B={B} H={H} L={L} non-causal", flush=True)
    monkeypatch.setenv("FAQ_ATTN_PACE", "0")
    ref = _run(qh, kh, vt, L, False)
    monkeypatch.delenv("FAQ_ATTN_PACE")
    for rep in range(2):
        got = _run(qh, kh, vt, L, False)
        print(f"[pace] launch {rep}", flush=True)
        assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])
