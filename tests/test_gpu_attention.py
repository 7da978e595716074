"""GPU parity of the HiF4 QK/PV attention kernel against the oracle and the reference goldens.

Tolerances (fp32 math).  The kernel's P-hat codes equal the reference quantizer's on the
kernel's own P bit for bit (tests/test_gpu_pquant.py), but that P comes from a hardware
exp2 on log2-scaled scores summed in MFMA order, the oracle's from numpy exp on BLAS-order
sums, so P differs by a few ulp, and where a P lies on a code boundary its code flips: one
flip moves an output row by one HiF4 step of one key's weight.  Each test therefore carries
its own bar, about ten times the error it reaches (measured on MI355X, the figure beside
each constant):
- TIGHT: paths with no code flips in the tested rows (the shape cases, levels, config 1,
  flags off, decode, chunked prefill): relative Frobenius 1e-5, max 1e-4 of the output's
  largest magnitude (reached: 2e-7 / 2e-6);
- FLIPS: inputs drawn with large scores (x2-x3 queries, masks, softcaps, mixed levels,
  random configurations, goldens), where flips are seen: 1e-3 / 1e-2 (reached: 1.4e-4 /
  5e-3 in the unquantized-normalizer random cases; the reference measured its own Triton
  kernel at 4-7e-4 relative error against its simulator, docs/WAN22.md:172-175).
The full-size bars are per configuration (tests/test_gpu_full_size.py).  Identities
(constant V under P-Reordering, fused == unfused prologue) are checked to a few ulps or
bitwise, and rows that see a single key bitwise (tests/test_gpu_single_key.py).
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from oracle import attention as OA
from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.golden.cases import CASES, build_inputs, golden_output

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FRO_TOL = 1e-3  # the FLIPS bar (module docstring)
MAX_TOL = 1e-2
TIGHT = dict(fro_tol=1e-5, max_tol=1e-4)


def to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(dtype)


def assert_close_attention(got: np.ndarray, ref: np.ndarray, what: str = "", *, fro_tol: float = FRO_TOL,
                           max_tol: float = MAX_TOL):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    assert np.isfinite(got).all()
    scale = max(np.abs(ref).max(), 1e-30)
    fro = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    mx = np.abs(got - ref).max() / scale
    print(f"[parity] {what} fro_rel={fro:.3e} max_rel={mx:.3e}", flush=True)
    assert fro <= fro_tol, (what, fro, fro_tol)
    assert mx <= max_tol, (what, mx, max_tol)


def module(*, qk=True, pv=True, mode="quantized_same", causal=True, query_chunk=256, key_chunk=128):
    from faquant_amd.simulated_flash_attention import new_simulated_attention_stats

    return SimpleNamespace(
        is_causal=causal,
        training=False,
        faquant_attention_query_chunk_size=query_chunk,
        faquant_attention_key_chunk_size=key_chunk,
        faquant_qk_matmul_quant=qk,
        faquant_pv_matmul_quant=pv,
        faquant_pv_normalizer_mode=mode,
        faquant_matmul_quant_kwargs={"quant_format": "hif4", "bits": 4, "group_size": 64,
                                     "symmetric": True, "clip_ratio": 1.0},
        faquant_simulated_attention_stats=new_simulated_attention_stats(),
    )


def with_levels(levels):
    """Temporarily set every attention operand's HiF4 levels (the env-derived table)."""
    from faquant_amd import hif4 as H

    class _Ctx:
        def __enter__(self):
            self.saved = dict(H.HIF4_ATTN_OPERAND_SCALE_LEVELS)
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.update(dict.fromkeys("qkpv", levels))

        def __exit__(self, *exc):
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.clear()
            H.HIF4_ATTN_OPERAND_SCALE_LEVELS.update(self.saved)

    return _Ctx()


@pytest.mark.parametrize("case", list(CASES))
def test_golden_cases_through_drop_in(dev, golden_attention, case):
    from faquant_amd.qwen3 import post_rope_qk_transform
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    builder, mk, _, levels, rot = CASES[case]
    q, k, v, dt = build_inputs(builder)
    tdt = torch.bfloat16 if dt == "bfloat16" else torch.float32
    qt, kt, vt = (to_dev(a, dev, tdt) for a in (q, k, v))
    if rot is not None:
        qt, kt = post_rope_qk_transform(qt, kt, rotation=True, rotation_block_size=rot)
    mod = module(qk=mk["qk"], pv=mk["pv"], mode=mk["mode"], causal=mk.get("causal", True))
    with with_levels(levels):
        out, w = simulated_flash_attention_forward(mod, qt, kt, vt, None)
    assert w is None and out.dtype == tdt and out.shape == (q.shape[0], q.shape[2], q.shape[1], q.shape[3])
    got = out.float().cpu().numpy()
    ref = golden_output(golden_attention, case)
    if case == "c1_unq":
        got = got[:, :, :4]
    assert_close_attention(got, ref, f"golden {case}")
    keys = [str(s) for s in golden_attention[f"{case}__stats_keys"]]
    stats = mod.faquant_simulated_attention_stats
    assert {kk: stats[kk] for kk in keys} == dict(zip(keys, golden_attention[f"{case}__stats"].tolist()))


def _oracle(q, k, v, *, causal=True, levels="123", mode="quantized_same", qk=True, pv=True, dtype="float32"):
    cfg = OA.SimConfig(qk_quant=qk, pv_quant=pv, pv_normalizer_mode=mode, levels=dict.fromkeys("qkpv", levels),
                       is_causal=causal)
    return OA.simulated_flash_attention(q, k, v, cfg, dtype=dtype)


def _kernel(dev, q, k, v, *, causal=True, levels="123", mode="quantized_same", qk=True, pv=True, out_dtype=torch.float32):
    from faquant_amd import _ops

    qt, kt, vt_ = (to_dev(a, dev, torch.bfloat16) for a in (q, k, v))
    qh, _ = _ops.operand_prep(qt, levels=levels if qk else None)
    kh, _ = _ops.operand_prep(kt, levels=levels if qk else None)
    vt = _ops.operand_prep_vt(vt_, levels=levels if pv else None)
    B, Hq, Lq, D = q.shape
    out = torch.empty((B, Lq, Hq, D), device=dev, dtype=out_dtype)
    _ops.attention_fwd(qh, kh, vt, k.shape[2], causal=causal, scale=D**-0.5, quant_p=pv, p_levels=levels,
                       norm_same=mode == "quantized_same", out=out.transpose(1, 2))
    return out.float().cpu().numpy()


SHAPES = [
    # (B, Hq, Hkv, Lq, Lk, causal)
    (1, 4, 1, 384, 384, True),
    (1, 2, 2, 130, 300, True),     # chunked prefill, ragged
    (1, 2, 1, 200, 70, True),      # more queries than keys: first rows see nothing
    (2, 6, 2, 97, 97, True),       # batch 2, GQA 3 (one head per workgroup)
    (1, 8, 1, 160, 160, True),     # GQA 8
    (1, 4, 2, 64, 64, True),       # GQA 2
    (1, 3, 3, 257, 333, False),    # non-causal MHA, ragged
    (1, 1, 1, 1, 129, True),       # a single query row
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("mode", ["quantized_same", "unquantized"])
def test_kernel_matches_oracle_fp32_out(dev, shape, mode):
    B, Hq, Hkv, Lq, Lk, causal = shape
    g = OI.rng(sum(shape))
    q = OQ.bf16_round(g.standard_normal((B, Hq, Lq, 128), dtype=np.float32) * 2)
    k = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((B, Hkv, Lk, 128), dtype=np.float32))
    got = _kernel(dev, q, k, v, causal=causal, mode=mode)
    ref = _oracle(q, k, v, causal=causal, mode=mode)
    assert_close_attention(got, ref, f"{shape} {mode}", **TIGHT)
    if causal and Lq > Lk:
        assert np.count_nonzero(got[:, : Lq - Lk]) == 0


@pytest.mark.parametrize("levels", ["12", "13"])
def test_p_levels_variants(dev, levels):
    q, k, v = OI.qwen(5, 4, 1, 256, student_t_keys=True)
    assert_close_attention(_kernel(dev, q, k, v, levels=levels), _oracle(q, k, v, levels=levels), f"levels {levels}",
                           **TIGHT)


@pytest.mark.parametrize("qk,pv", [(True, False), (False, True), (False, False)])
def test_quantization_flags(dev, qk, pv):
    q, k, v = OI.qwen(6, 4, 1, 256)
    mode = "unquantized"
    assert_close_attention(_kernel(dev, q, k, v, qk=qk, pv=pv, mode=mode),
                           _oracle(q, k, v, qk=qk, pv=pv, mode=mode), f"qk={qk} pv={pv}", **TIGHT)


def test_constant_values_are_reproduced_under_p_reordering(dev):
    """V = 1 (V^ = HiF4(1) = 0.9375 for a constant block): under quantized_same numerator and
    denominator sum the same P^, so every output is V^ up to fp32 rounding of the two sums
    and their running-max rescales (a few ulps)
    (the reference's int-format version of this test is exact: 1 stays 1 there)."""
    g = OI.rng(9)
    q = OQ.bf16_round(g.standard_normal((1, 4, 700, 128), dtype=np.float32) * 3)
    k = OQ.bf16_round(g.standard_normal((1, 2, 700, 128), dtype=np.float32) * 3)
    v = np.ones((1, 2, 700, 128), np.float32)
    vhat = float(OQ.fake_quantize_hif4(v[0, 0, :1], "123")[0, 0])
    assert vhat == 0.9375
    got = _kernel(dev, q, k, v, mode="quantized_same")
    np.testing.assert_allclose(got, vhat, rtol=1e-6, atol=0)
    mism = _kernel(dev, q, k, v, mode="unquantized")
    assert np.abs(mism - vhat).max() > 1e-3


def test_constant_scores_average_values(dev):
    """Q = 0: every allowed P is 1, P^ is one constant, so row p returns mean(V^[:p+1])."""
    g = OI.rng(10)
    L = 300
    q = np.zeros((1, 2, L, 128), np.float32)
    k = OQ.bf16_round(g.standard_normal((1, 1, L, 128), dtype=np.float32))
    v = OQ.bf16_round(g.standard_normal((1, 1, L, 128), dtype=np.float32))
    got = _kernel(dev, q, k, v, mode="quantized_same")
    vq = OQ.fake_quantize_hif4(v, "123").astype(np.float64)[0, 0]
    expect = np.cumsum(vq, axis=0) / np.arange(1, L + 1)[:, None]
    np.testing.assert_allclose(got[0, :, 0], expect, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got[0, :, 1], expect, rtol=1e-5, atol=1e-5)


def test_config1_full(dev):
    """Configuration 1: fp32, 8 heads, L=512, causal, outlier channels, both modes."""
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = OI.config1()
    for mode in ("quantized_same", "unquantized"):
        out, _ = simulated_flash_attention_forward(module(mode=mode), to_dev(q, dev), to_dev(k, dev), to_dev(v, dev), None)
        assert out.dtype == torch.float32
        assert_close_attention(out.cpu().numpy(), _oracle(q, k, v, mode=mode), f"config1 {mode}", **TIGHT)


def test_wan_hif4_attention_drop_in(dev):
    from faquant_amd.wan22_attention import hif4_attention

    q, k, v = OI.wan(12, 3, 333)
    qq, kq, vq = (OQ.fake_quantize_hif4(a, "123", "bfloat16") for a in (q, k, v))
    for norm in (False, True):
        out = hif4_attention(to_dev(qq[0], dev, torch.bfloat16), to_dev(kq[0], dev, torch.bfloat16),
                             to_dev(vq[0], dev, torch.bfloat16), quantized_normalizer=norm)
        assert out.shape == (333, 3, 128) and out.dtype == torch.bfloat16
        t = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
        # the oracle quantizes the raw V itself: HiF4 QDQ is not idempotent, so V^ must not be re-quantized
        ref = _oracle(t(qq), t(kq), t(v), causal=False, qk=False, mode="quantized_same" if norm else "unquantized",
                      dtype="bfloat16")
        assert_close_attention(out.float().cpu().numpy(), ref[0], f"hif4_attention norm={norm}")


def test_make_flash_attention_fused_equals_unfused(dev):
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.wan22_attention import faquant_qdq, make_flash_attention

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in OI.wan(13, 2, 260))
    q2 = torch.cat([q, q.flip(1)])  # batch 2
    k2 = torch.cat([k, k.flip(1)])
    v2 = torch.cat([v, v.flip(1)])
    for rot in (False, True):
        fused = make_flash_attention(faquant_qdq("123"), quantized_normalizer=True, qk_rotation=rot)
        plain = make_flash_attention(lambda t: fake_quantize_hif4(t, levels="123"), quantized_normalizer=True,
                                     qk_rotation=rot)
        a = fused(q2, k2, v2)
        b = plain(q2, k2, v2)
        assert a.shape == q2.shape
        assert torch.equal(a, b)
    # and the whole recipe against the oracle (rotation -> bf16 -> QDQ -> attention)
    qn, kn, vn = (t.float().cpu().numpy()[0].transpose(1, 0, 2)[None] for t in (q, k, v))
    qr = OQ.bf16_round(OH.hadamard_transform(qn))
    kr = OQ.bf16_round(OH.hadamard_transform(kn))
    ref = _oracle(qr, kr, vn, causal=False, dtype="bfloat16")
    assert_close_attention(a[0].float().cpu().numpy(), ref[0], "wan recipe")


def test_qwen_attention_core_equals_two_step(dev):
    """qwen3.attention_core (fused prologue) == post_rope_qk_transform + simulated forward, bitwise."""
    from faquant_amd.qwen3 import attention_core, post_rope_qk_transform
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q, k, v = (to_dev(a, dev, torch.bfloat16) for a in OI.qwen(14, 8, 2, 300))
    g = OI.rng(15)
    scale = to_dev(g.uniform(0.5, 2.0, size=(128,)), dev)
    offset = to_dev(g.standard_normal((2, 1, 128)) * 0.3, dev)
    for block in (None, 64):
        mod = module()
        mod.faquant_qk_smooth_scale = scale
        mod.faquant_qk_key_offset = offset
        mod.faquant_qk_rotation = True
        mod.faquant_qk_rotation_block_size = block
        fused = attention_core(mod, q, k, v)
        qr, kr = post_rope_qk_transform(q, k, smooth_scale=scale, key_offset=offset, rotation=True,
                                        rotation_block_size=block)
        two, _ = simulated_flash_attention_forward(module(), qr, kr, v, None)
        assert torch.equal(fused, two)


def test_hif4_sign_symmetry_and_power_of_two_equivariance(dev):
    """QDQ(-x) = -QDQ(x), and QDQ(2^j x) = 2^j QDQ(x) away from the scale clamps.
    (QDQ is not idempotent: a block of ones maps to 0.9375, whose own scale is smaller.)"""
    from faquant_amd.hif4 import fake_quantize_hif4

    x = torch.randn(4096, 128, device=dev)
    y = fake_quantize_hif4(x, levels="123")
    assert torch.equal(fake_quantize_hif4(-x, levels="123"), -y)
    for j in (-20, -3, 5, 11):
        assert torch.equal(fake_quantize_hif4(x * 2.0**j, levels="123"), y * 2.0**j)
    ones = torch.ones(1, 64, device=dev)
    assert fake_quantize_hif4(ones, levels="123")[0, 0].item() == 0.9375
    assert fake_quantize_hif4(fake_quantize_hif4(ones, levels="123"), levels="123")[0, 0].item() == 0.875


def test_unsupported_features_raise(dev):
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward

    q = torch.randn(1, 2, 8, 128, device=dev)
    k = torch.randn(1, 1, 8, 128, device=dev)
    with pytest.raises(NotImplementedError, match="key chunks"):
        simulated_flash_attention_forward(module(key_chunk=4096), q, k, k, None)
    mod = module()
    mod.faquant_matmul_quant_kwargs = dict(mod.faquant_matmul_quant_kwargs, quant_format="int")
    with pytest.raises(NotImplementedError, match="quant_format"):
        simulated_flash_attention_forward(mod, q, k, k, None)
    wide = torch.randn(1, 1, 8, 512, device=dev)
    with pytest.raises(NotImplementedError, match="head_dim"):
        simulated_flash_attention_forward(module(), wide, wide, wide, None)
    # an all-valid mask is the mask-free case
    out_m, _ = simulated_flash_attention_forward(module(), q, k, k, torch.ones(1, 8, dtype=torch.bool, device=dev))
    out_n, _ = simulated_flash_attention_forward(module(), q, k, k, None)
    assert torch.equal(out_m, out_n)


def test_forward_only_paths_join_autograd_and_refuse_backward(dev):
    """The reference's simulator is differentiable (test_simulated_flash_attention.py:818-876);
    this build implements inference.  With inputs that require grad, each drop-in returns
    the no-grad result joined to the autograd graph, and a backward pass through it raises
    instead of silently leaving those inputs without a gradient."""
    from faquant_amd.quantization import FakeQuantLinear
    from faquant_amd.simulated_flash_attention import simulated_flash_attention_forward
    from faquant_amd.wan22_attention import hif4_attention

    g = torch.Generator(device="cpu").manual_seed(3)
    q, k, v = (torch.randn(1, h, 200, 128, generator=g).to(dev, torch.bfloat16) for h in (4, 2, 2))
    with torch.no_grad():
        ref, _ = simulated_flash_attention_forward(module(), q, k, v, None)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    out, _ = simulated_flash_attention_forward(module(), qg, kg, vg, None)
    assert out.requires_grad and torch.equal(out.detach(), ref)
    with pytest.raises(NotImplementedError, match="forward-only"):
        out.float().sum().backward()

    ql, kl, vl = (t[0, :2].transpose(0, 1).contiguous().requires_grad_(True) for t in (q, k, v))
    wan = hif4_attention(ql, kl, vl)
    assert wan.requires_grad
    with pytest.raises(NotImplementedError, match="forward-only"):
        wan.float().sum().backward()

    lin = torch.nn.Linear(128, 64).to(dev, torch.bfloat16)
    mod = FakeQuantLinear(lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64,
                          symmetric=True, clip_ratio=1.0)
    x = torch.randn(8, 128, generator=g).to(dev, torch.bfloat16).requires_grad_(True)
    y = mod(x)
    assert y.requires_grad
    with pytest.raises(NotImplementedError, match="forward-only"):
        y.float().sum().backward()
    with torch.no_grad():  # inference mode: plain tensors, nothing tracked
        assert not simulated_flash_attention_forward(module(), qg, kg, vg, None)[0].requires_grad
