"""The C ABI boundary and the host-side mirror, without a GPU.

* libfaquant_amd.so loads and exports every entry point include/faquant_amd.h declares;
* argument validation returns the documented status before any device work;
* the drop-in Python functions raise the reference's exception types and
  messages for invalid arguments, and refuse CPU tensors (no CPU fallback).
"""

import ctypes
import os
import re
from types import SimpleNamespace

import pytest

from tests.conftest import REPO

torch = pytest.importorskip("torch")

HEADER = os.path.join(REPO, "include", "faquant_amd.h")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w[\w\s\*]*?\b(faq_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from faquant_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("HIP library not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_lists_the_entry_points():
    names = declared()
    assert names == sorted(
        ["faq_last_error", "faq_version", "faq_hif4_qdq_rows", "faq_hif4_unpack_rows", "faq_hadamard_rows",
         "faq_act_qdq_rows", "faq_operand_prep", "faq_operand_prep_vt", "faq_attention_fwd",
         "faq_attention_fwd_split", "faq_attention_split_workspace", "faq_attention_mask_bounds",
         "faq_mfma_probe", "faq_stream_probe", "faq_pquant_groups", "faq_hadamard_rows_native", "faq_attention_fwd_split_noalloc",
         "faq_operand_prep_hif4_kv", "faq_attention_decode", "faq_attention_decode_workspace",
         "faq_act_prep_rows", "faq_act_compand_rcp", "faq_hif4_linear_packed", "faq_attention_fwd_general"]
    )


def test_library_exports_every_declared_symbol(lib):
    from faquant_amd import _lib

    for name in declared():
        assert hasattr(lib, name), name
    assert set(declared()) == set(_lib.EXPORTED)
    assert lib.faq_version().decode().startswith("faquant_amd")


def test_validation_statuses_without_device_work(lib):
    from faquant_amd import _lib

    assert lib.faq_hif4_qdq_rows(None, None, 1, 64, 0, 123, *([None] * 8), None) == _lib.EINVAL
    assert "null" in lib.faq_last_error().decode()
    buf = ctypes.create_string_buffer(1024)
    p = ctypes.addressof(buf)
    p16 = (p + 15) // 16 * 16
    assert lib.faq_hif4_qdq_rows(p16, p16, 1, 64, 0, 7, *([None] * 8), None) == _lib.EINVAL
    assert "123, 12 or 13" in lib.faq_last_error().decode()
    assert lib.faq_mfma_probe(None, 1, 1, None) == _lib.EINVAL
    assert lib.faq_mfma_probe(p16, 0, 1, None) == _lib.EINVAL
    assert lib.faq_stream_probe(None, 16, p16, 1, None) == _lib.EINVAL
    assert lib.faq_stream_probe(p16, 24, p16, 1, None) == _lib.EINVAL
    assert lib.faq_stream_probe(p16, 16, p16, 0, None) == _lib.EINVAL
    assert lib.faq_hadamard_rows(p16, p16, 1, 24, 3, 0, 0, None) == _lib.EINVAL
    assert "power of two" in lib.faq_last_error().decode()
    assert lib.faq_act_qdq_rows(p16, p16, 1, 96, 1, None, 64, 123, None) == _lib.EINVAL
    assert "divisible by power-of-two block_size=64" in lib.faq_last_error().decode()
    assert lib.faq_act_qdq_rows(p16, p16, 1, 64, 1, None, 0, 99, None) == _lib.EINVAL
    assert "123, 12 or 13" in lib.faq_last_error().decode()
    assert lib.faq_act_qdq_rows(p16, p16, 1, 12, 1, None, 0, 123, None) == _lib.EUNSUP
    # the full activation path: rows of at most 32768 features, a rotation needs signs and permutation,
    # block sizes are powers of two dividing the row, levels 0 (no quantizer) or 123 / 12 / 13
    ao = _lib.ActOpts()
    assert lib.faq_act_prep_rows(p16, p16, 1, 96, 1, None, 123, None) == _lib.EUNSUP
    assert lib.faq_act_prep_rows(p16, p16, 1, 32768 + 64, 1, None, 123, None) == _lib.EUNSUP
    assert lib.faq_act_prep_rows(p16, p16, 1, 64, 1, None, 99, None) == _lib.EINVAL
    assert lib.faq_act_prep_rows(p16 + 2, p16, 1, 64, 1, None, 123, None) == _lib.EINVAL
    ao.rot_signs = p16
    assert lib.faq_act_prep_rows(p16, p16, 1, 128, 1, ctypes.byref(ao), 123, None) == _lib.EINVAL
    assert "signs and permutation" in lib.faq_last_error().decode()
    ao.rot_perm = p16
    ao.rot_block = 96
    assert lib.faq_act_prep_rows(p16, p16, 1, 192, 1, ctypes.byref(ao), 123, None) == _lib.EINVAL
    assert "power of two" in lib.faq_last_error().decode()
    ao.rot_block = 0
    ao.hadamard = 256
    assert lib.faq_act_prep_rows(p16, p16, 1, 192, 1, ctypes.byref(ao), 0, None) == _lib.EINVAL
    assert "divisible by power-of-two block_size=256" in lib.faq_last_error().decode()
    ao = _lib.ActOpts()
    ao.rot_perm = p16
    assert lib.faq_act_prep_rows(p16, p16, 1, 128, 1, ctypes.byref(ao), 123, None) == _lib.EINVAL
    ao = _lib.ActOpts()
    ao.compand = p16 + 4  # the kernel reads the per-feature vectors 16 bytes at a time
    assert lib.faq_act_prep_rows(p16, p16, 1, 128, 1, ctypes.byref(ao), 123, None) == _lib.EINVAL
    assert "16-byte aligned" in lib.faq_last_error().decode()
    assert lib.faq_act_prep_rows(p16, p16, 0, 128, 1, None, 123, None) == _lib.OK
    # an empty batch (torch gives its storage a null pointer) launches nothing
    assert lib.faq_act_prep_rows(None, None, 0, 128, 1, None, 123, None) == _lib.OK
    assert lib.faq_act_qdq_rows(None, None, 0, 128, 1, None, 0, 123, None) == _lib.OK
    assert lib.faq_act_prep_rows(None, None, 1, 128, 1, None, 123, None) == _lib.EINVAL
    assert lib.faq_hif4_qdq_rows(None, None, 0, 64, 1, 123, *([None] * 8), None) == _lib.OK
    assert lib.faq_hadamard_rows(None, None, 0, 128, 64, 1, 1, None) == _lib.OK
    assert lib.faq_hadamard_rows(p16, p16, -1, 128, 64, 1, 1, None) == _lib.EINVAL
    assert lib.faq_hadamard_rows_native(None, None, 0, 128, 1, None) == _lib.OK
    assert lib.faq_operand_prep(p16, 1, 128, 128, 128, 1, 1, 1, None, 0, None, 0, 0, 96, 1, None, p16, 128, 128, 128,
                                123, None) == _lib.EUNSUP
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 128, p16, 1, 0, 0, 0,
                               1, 3, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 0, None, None)
    assert rc == _lib.EINVAL and "divisible" in lib.faq_last_error().decode()
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 100, p16, 1, 0, 0, 0,
                               1, 2, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 0, None, None)
    assert rc == _lib.EINVAL and "Lpad" in lib.faq_last_error().decode()
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 128, p16, 1, 0, 0, 0,
                               1, 2, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 45, None, None)
    assert rc == _lib.EINVAL and "123, 12 or 13" in lib.faq_last_error().decode()
    # score options: ranges and key bits go together; the softcap needs the ranges
    opts = _lib.AttnOpts()
    opts.row_lo = p16
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 128, p16, 1, 0, 0, 0,
                               1, 2, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 0, ctypes.byref(opts), None)
    assert rc == _lib.EINVAL and "go together" in lib.faq_last_error().decode()
    opts = _lib.AttnOpts()
    opts.softcap = 30.0
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 128, p16, 1, 0, 0, 0,
                               1, 2, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 0, ctypes.byref(opts), None)
    assert rc == _lib.EINVAL and "softcap needs key ranges" in lib.faq_last_error().decode()
    opts.softcap = -1.0
    rc = lib.faq_attention_fwd(p16, 0, 0, 0, p16, 0, 0, 0, p16, 0, 0, 128, 128, p16, 1, 0, 0, 0,
                               1, 2, 2, 1, 1, 1, 0.1, 1, 123, 1, None, 0, ctypes.byref(opts), None)
    assert rc == _lib.EINVAL and "non-negative" in lib.faq_last_error().decode()
    assert lib.faq_attention_mask_bounds(None, 0, 1, 4, 4, 1, 0, None, None, None, None, 0, None) == _lib.EINVAL
    assert lib.faq_attention_mask_bounds(None, 0, 1, 4, 4, 1, -2, p16, p16, p16, None, 0, None) == _lib.EINVAL
    assert "sliding_window" in lib.faq_last_error().decode()
    assert lib.faq_attention_mask_bounds(None, 0, 1, 4, 1 << 20, 1, 0, p16, p16, p16, None, 0, None) == _lib.EUNSUP
    assert lib.faq_attention_mask_bounds(None, 0, 1, 4, 300, 1, 0, p16, p16, p16, p16, 8, None) == _lib.EINVAL
    assert "key_words" in lib.faq_last_error().decode()


def test_general_attention_validation_without_device_work(lib):
    """faq_attention_fwd_general refuses bad sizes and types before touching the device."""
    from faquant_amd import _lib

    def call(B=1, Hq=2, Hkv=1, Lq=4, Lk=4, D=64, tile=128, dt=_lib.F32, levels=123, quant_p=1, p=1):
        ptr = p if p else None
        return lib.faq_attention_fwd_general(ptr, dt, 0, 0, 0, ptr, dt, 0, 0, 0, ptr, dt, 0, 0, 0, ptr, dt, 0, 0, 0,
                                             B, Hq, Hkv, Lq, Lk, D, tile, 1, 0.125, quant_p, levels, 1, None, None,
                                             None)

    assert call(D=0) == _lib.EUNSUP and "head_dim" in lib.faq_last_error().decode()
    assert call(D=257) == _lib.EUNSUP
    assert call(tile=0) == _lib.EUNSUP and "key tiles" in lib.faq_last_error().decode()
    assert call(tile=1025) == _lib.EUNSUP
    assert call(Hq=3, Hkv=2) == _lib.EINVAL
    assert call(dt=7) == _lib.EUNSUP
    assert call(levels=7) == _lib.EINVAL
    assert call(p=0) == _lib.EINVAL and "null" in lib.faq_last_error().decode()
    assert call(B=0) == _lib.OK and call(Lq=0) == _lib.OK  # empty: nothing launched


def test_status_maps_to_reference_exception_types(lib):
    from faquant_amd import _lib

    lib.faq_hadamard_rows(None, None, 1, 8, 8, 0, 0, None)
    with pytest.raises(ValueError):
        _lib.check(_lib.EINVAL)
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.EUNSUP)


def _module():
    from faquant_amd.simulated_flash_attention import new_simulated_attention_stats

    return SimpleNamespace(
        is_causal=True, training=False, faquant_attention_query_chunk_size=256,
        faquant_attention_key_chunk_size=128, faquant_qk_matmul_quant=True, faquant_pv_matmul_quant=True,
        faquant_pv_normalizer_mode="quantized_same",
        faquant_matmul_quant_kwargs={"quant_format": "hif4", "bits": 4, "group_size": 64, "symmetric": True,
                                     "clip_ratio": 1.0},
        faquant_simulated_attention_stats=new_simulated_attention_stats(),
    )


def test_drop_in_validation_messages_match_reference():
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward as f

    q = torch.zeros(1, 2, 3, 128)
    k = torch.zeros(1, 1, 3, 128)
    with pytest.raises(ValueError, match="dropout=0"):
        f(_module(), q, k, k, None, dropout=0.1)
    with pytest.raises(ValueError, match="rank-4"):
        f(_module(), q[0], k, k, None)
    with pytest.raises(ValueError, match="matching K/V"):
        f(_module(), q, k, torch.zeros(1, 1, 4, 128), None)
    with pytest.raises(ValueError, match="divisible"):
        f(_module(), torch.zeros(1, 3, 3, 128), torch.zeros(1, 2, 3, 128), torch.zeros(1, 2, 3, 128), None)
    with pytest.raises(NotImplementedError, match="packed cu_seqlens"):
        f(_module(), q, k, k, None, cu_seq_lens_q=torch.tensor([0, 3]))
    with pytest.raises(ValueError, match="sliding_window must be positive"):
        f(_module(), q, k, k, None, sliding_window=0)
    mod = _module()
    mod.faquant_pv_normalizer_mode = "quantized"
    with pytest.raises(ValueError, match="pv_normalizer_mode"):
        f(mod, q, k, k, None)


def test_cpu_tensors_are_refused_not_computed(lib):
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward as f

    with pytest.raises(ValueError, match="ROCm device"):
        fake_quantize_hif4(torch.zeros(4, 64))
    with pytest.raises(ValueError, match="ROCm device"):
        f(_module(), torch.zeros(1, 2, 3, 128), torch.zeros(1, 1, 3, 128), torch.zeros(1, 1, 3, 128), None)


def test_quantizer_argument_errors():
    from faquant_amd.hif4 import fake_quantize_hif4, fit_hif4_compact_parameters
    from faquant_amd.quantization import fake_quantize

    with pytest.raises(TypeError, match="floating-point"):
        fake_quantize_hif4(torch.zeros(4, 64, dtype=torch.int32))
    with pytest.raises(ValueError, match="at least one dimension"):
        fit_hif4_compact_parameters(torch.tensor(1.0))
    with pytest.raises(ValueError, match="final dimension of 64"):
        fit_hif4_compact_parameters(torch.zeros(2, 32))
    with pytest.raises(ValueError, match="bits=4"):
        fake_quantize(torch.zeros(2, 64), quant_format="hif4", bits=8)
    with pytest.raises(ValueError, match="group_size=64"):
        fake_quantize(torch.zeros(2, 64), quant_format="hif4", group_size=32)
    with pytest.raises(NotImplementedError):
        fake_quantize(torch.zeros(2, 64), quant_format="int", bits=4, group_size=4)


def test_stats_closed_form_matches_oracle_counters():
    """count_tiles replays the simulator schedule: compare with the oracle's counters."""
    import numpy as np

    from faquant_amd.simulated_flash_attention import count_tiles, new_simulated_attention_stats
    from oracle import attention as OA

    for (B, Hq, Hkv, Lq, Lk, qc, causal) in ((1, 4, 2, 300, 300, 256, True), (2, 2, 1, 130, 400, 64, True),
                                              (1, 2, 2, 200, 200, 256, False), (1, 2, 1, 9, 3, 4, True)):
        q = np.zeros((B, Hq, Lq, 128), np.float32)
        k = np.zeros((B, Hkv, Lk, 128), np.float32)
        so = OA.new_stats()
        OA.simulated_flash_attention(q, k, k, OA.SimConfig(query_chunk=qc), is_causal=causal, stats=so)
        sg = new_simulated_attention_stats()
        count_tiles(sg, batch=B, query_heads=Hq, query_length=Lq, key_length=Lk, head_dim=128, query_chunk=qc,
                    key_chunk=128, causal=causal, skip_fully_masked=True, qk_quant=True, pv_quant=True,
                    qk_group=64, pv_group=64)
        assert sg == so


def test_split_count_rule():
    """Decode-sized grids split the key tiles so each CU holds one work item; prefill-sized
    query blocks, full grids and key lengths past the split path's tile limit do not split."""
    from faquant_amd import _ops

    # Qwen3-8B decode: 8 work items on 256 CUs -> 32 ranges, at most one per key tile
    assert [_ops._split_count(1, 32, 8, 1, lk) for lk in (1024, 4096, 32768, 131072)] == [8, 32, 32, 32]
    assert _ops._split_count(1, 32, 8, 1, 300) == 1                       # under four key tiles
    assert _ops._split_count(1, 32, 8, 65, 32768) == 1                    # a prefill chunk
    assert _ops._split_count(32, 32, 8, 1, 32768) == 1                    # 256 items fill the GPU
    assert _ops._split_count(16, 32, 8, 1, 32768) == 2                    # 128 items: two ranges
    assert _ops._split_count(1, 32, 8, 1, 32768, cus=80) == 10            # fewer CUs, fewer ranges
    assert _ops._split_count(1, 32, 8, 1, (_ops.SPLIT_MAX_TILES + 1) * 128) == 1


def test_decode_split_count_rule():
    """Key ranges of the decode kernel: about eight waves per CU, one tile per range at
    short contexts, two tiles per range where four waves per CU remain (bf16 K/V), no empty
    range."""
    from faquant_amd import _ops

    # Qwen3-8B heads (8 KV heads) on 256 CUs
    assert _ops.decode_split_count(1, 8, 8192) == 64        # 64 tiles, one each
    assert _ops.decode_split_count(1, 8, 32768) == 128      # 256 tiles, two each: 1024 waves
    assert _ops.decode_split_count(1, 8, 131072) == 256     # 1024 tiles, four each
    assert _ops.decode_split_count(1, 8, 5000) == 40        # 40 tiles (ragged last), one each
    assert _ops.decode_split_count(1, 8, 0) == 1
    # packed K/V keep one tile per range
    assert _ops.decode_split_count(1, 8, 32768, packed=True) == 256
    assert _ops.decode_split_count(1, 8, 131072, packed=True) == 256
    for b, lk in ((1, 300), (4, 32768), (32, 131072), (1, 2_000_000)):
        n = _ops.decode_split_count(b, 8, lk)
        tiles = -(-lk // 128)
        tps = -(-tiles // n)
        assert 1 <= n <= 4096 and (n - 1) * tps < tiles  # every range holds a tile


def test_attention_core_validates_like_the_drop_in():
    from faquant_amd.qwen3 import attention_core

    q, k = torch.zeros(1, 2, 3, 128, dtype=torch.bfloat16), torch.zeros(1, 1, 3, 128, dtype=torch.bfloat16)
    mod = _module()
    mod.faquant_pv_normalizer_mode = "quantized"
    with pytest.raises(ValueError, match="pv_normalizer_mode"):
        attention_core(mod, q, k, k)
    with pytest.raises(ValueError, match="sliding_window must be positive"):
        attention_core(_module(), q, k, k, sliding_window=0)


def test_pquant_groups_validation(lib):
    from faquant_amd import _lib

    assert lib.faq_pquant_groups(None, None, 1, 123, None) == _lib.EINVAL
    assert lib.faq_pquant_groups(None, None, 1, 7, None) == _lib.EINVAL
    assert "levels" in lib.faq_last_error().decode()
    assert lib.faq_pquant_groups(None, None, 0, 123, None) == _lib.OK
    assert lib.faq_hadamard_rows_native(None, None, 1, 128, 1, None) == _lib.EINVAL
    p16 = ctypes.c_void_p(1 << 20)
    assert lib.faq_hadamard_rows_native(p16, p16, 1, 96, 1, None) == _lib.EINVAL
    assert lib.faq_hadamard_rows_native(p16, p16, 1, 1024, 1, None) == _lib.EUNSUP
    assert lib.faq_hadamard_rows_native(p16, p16, 1, 128, 0, None) == _lib.EINVAL


def test_packed_linear_validation(lib):
    """faq_hif4_linear_packed refuses bad arguments before any device work."""
    from faquant_amd import _lib

    p16 = ctypes.c_void_p(1 << 20)

    def linear(**kw):
        a = dict(x=p16, xs=4096, c=p16, m=p16, b=None, bd=0, y=p16, yd=1, ys=4096, M=1, N=4096, K=4096)
        a.update(kw)
        return lib.faq_hif4_linear_packed(a["x"], a["xs"], a["c"], a["m"], a["b"], a["bd"], a["y"], a["yd"], a["ys"],
                                          a["M"], a["N"], a["K"], None)

    assert linear(x=None) == _lib.EINVAL
    assert linear(K=4000, xs=4000) == _lib.EUNSUP
    assert "multiple of 128" in lib.faq_last_error().decode()
    assert linear(M=9) == _lib.EUNSUP
    assert "at most 8 rows" in lib.faq_last_error().decode()
    assert linear(N=0) == _lib.EINVAL
    assert linear(yd=2) == _lib.EUNSUP  # fp16 output
    assert linear(b=p16, bd=2) == _lib.EUNSUP  # fp16 bias
    assert linear(xs=4095) == _lib.EINVAL
    assert linear(ys=4095) == _lib.EINVAL
    assert linear(m=ctypes.c_void_p((1 << 20) + 4)) == _lib.EINVAL  # meta not 8-byte aligned
    assert linear(y=ctypes.c_void_p((1 << 20) + 2), yd=0) == _lib.EINVAL  # fp32 y not 4-byte aligned
    assert linear(M=0, x=None, y=None) == _lib.OK  # no rows: nothing to do


def test_decode_and_packed_prep_validation(lib):
    """faq_attention_decode / faq_operand_prep_hif4_kv refuse bad arguments before any device
    work (a non-null dummy pointer is never dereferenced on these paths)."""
    from faquant_amd import _lib

    p16 = ctypes.c_void_p(1 << 20)
    assert lib.faq_attention_decode_workspace(1, 32, 1, 5000, 0) == -1
    ws = lib.faq_attention_decode_workspace(1, 32, 1, 5000, 40)
    # S (32 rows x 40 tiles x 128 keys) + tile maxima + split maxima + partials, 256-aligned
    assert ws == 655360 + 10240 + 5120 + 655360 + 10240

    def decode(**kw):
        a = dict(q=p16, k=p16, vt=p16, kp=None, vp=None, o=p16, Hq=32, Hkv=8, Lq=1, Lk=5000, nsplit=40, ws=p16,
                 wsb=1 << 30, qp=1, lv=123, strides=(0, 0, 0))
        a.update(kw)
        s = a["strides"]
        return lib.faq_attention_decode(a["q"], *s, a["k"], *s, a["vt"], 0, 0, 5120, a["kp"], a["vp"], a["o"], 1,
                                        *s, 1, a["Hq"], a["Hkv"], a["Lq"], a["Lk"], 1, 0.088, a["qp"], a["lv"], 1,
                                        None, a["nsplit"], a["ws"], a["wsb"], None)

    kv = _lib.HiF4KV(1 << 20, 1 << 20, 0, 0)
    assert decode(q=None) == _lib.EINVAL
    assert decode(kp=ctypes.byref(kv)) == _lib.EINVAL  # K packed, V not
    assert "both packed" in lib.faq_last_error().decode()
    assert decode(Hq=33) == _lib.EINVAL
    assert decode(Hq=64, Hkv=1) == _lib.EUNSUP  # more than 32 query heads per KV head
    assert decode(nsplit=0) == _lib.EINVAL
    assert decode(nsplit=5000) == _lib.EINVAL
    assert decode(lv=7) == _lib.EINVAL
    assert decode(strides=(1, 0, 0)) == _lib.EINVAL
    assert decode(wsb=100) == _lib.EINVAL
    assert "workspace" in lib.faq_last_error().decode()
    assert decode(ws=None) == _lib.EINVAL
    bad = _lib.HiF4KV(1 << 20, (1 << 20) + 4, 0, 0)  # meta not 8-byte aligned
    assert decode(kp=ctypes.byref(bad), vp=ctypes.byref(kv)) == _lib.EINVAL
    assert decode(Lq=0) == _lib.OK  # nothing to do

    def prep(**kw):
        a = dict(x=p16, codes=p16, meta=p16, lv=123, had=0, dt=1)
        a.update(kw)
        return lib.faq_operand_prep_hif4_kv(a["x"], a["dt"], 0, 0, 128, 1, 1, 4, None, 0, None, 0, 0, a["had"], 1,
                                            a["lv"], a["codes"], a["meta"], 0, 0, None)

    assert prep(codes=None) == _lib.EINVAL
    assert prep(lv=0) == _lib.EINVAL  # the packed form needs HiF4 levels
    assert prep(had=32) == _lib.EUNSUP
    assert prep(dt=9) == _lib.EINVAL
    assert prep(meta=ctypes.c_void_p((1 << 20) + 4)) == _lib.EINVAL
