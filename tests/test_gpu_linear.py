"""HiF4 W4A4 Linear: the fused activation prologue and the Linear drop-ins.

The activation path of FakeQuantLinear.forward (quantization.py:199-276) is
x * dtype(input_scale) in the input dtype, the HiSQ input rotation, the clamp,
the companding product, the per-block fp32 Hadamard (rotation.py:117-135, true
division by sqrt(n)) cast back to the input dtype, fake_quantize (HiF4, ACT levels)
in that dtype and the companding quotient.  The oracles restate each step (pinned
against the reference's codec, Hadamard and FakeQuantLinear goldens), so the kernels
are compared with them bit for bit, and with the reference-written activations
directly; the Linear drop-ins are compared with the reference's composition of
those steps and F.linear.
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest

from oracle import hadamard as OH
from oracle import hif4 as OQ
from oracle import inputs as OI
from tests.test_gpu_attention import to_dev

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _round(x, dtype):
    return OQ.bf16_round(x) if dtype == torch.bfloat16 else np.asarray(x, np.float32)


def _oracle_act(x, dtype, *, scale=None, hadamard=0, levels="123"):
    name = "bfloat16" if dtype == torch.bfloat16 else "float32"
    v = np.asarray(x, np.float32)
    if scale is not None:
        v = _round(v * _round(scale, dtype), dtype)
    if hadamard:
        v = _round(OH.block_hadamard_transform(v, hadamard), dtype)
    return OQ.fake_quantize_hif4(v, levels, dtype=name) if levels else v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("hadamard", [0, 64, 128, 512])
@pytest.mark.parametrize("levels", ["123", "12", "13"])
def test_act_prologue_matches_oracle_bitwise(dev, dtype, hadamard, levels):
    from faquant_amd import _ops

    g = OI.rng(hadamard + int(levels))
    x = _round(g.standard_normal((37, 1024), dtype=np.float32) * np.exp(g.standard_normal((1, 1024))), dtype)
    x[3, 100:140] = 0.0  # zero groups
    scale = g.uniform(0.25, 4.0, size=(1024,)).astype(np.float32)
    for sc in (None, scale):
        got = _ops.act_qdq_rows(to_dev(x, dev, dtype), levels=levels, hadamard=hadamard,
                                col_scale=None if sc is None else to_dev(sc, dev))
        ref = _oracle_act(x, dtype, scale=sc, hadamard=hadamard, levels=levels)
        print(f"[act] {dtype} hadamard={hadamard} levels={levels} scale={sc is not None}", flush=True)
        assert np.array_equal(got.float().cpu().numpy(), ref)


def test_act_prologue_partial_group_and_leading_shape(dev):
    from faquant_amd import _ops

    g = OI.rng(7)
    x = OQ.bf16_round(g.standard_normal((2, 3, 200), dtype=np.float32))
    got = _ops.act_qdq_rows(to_dev(x, dev, torch.bfloat16), levels="123")
    assert got.shape == (2, 3, 200)
    assert np.array_equal(got.float().cpu().numpy(), OQ.fake_quantize_hif4(x, "123", dtype="bfloat16"))


@pytest.mark.parametrize("block", [None, 64])
def test_fake_quant_linear_equals_reference_composition(dev, block):
    from faquant_amd import _ops
    from faquant_amd.hif4 import HIF4_ACT_SCALE_LEVELS, HIF4_SCALE_LEVELS
    from faquant_amd.quantization import FakeQuantLinear, fake_quantize

    g = OI.rng(8)
    lin = torch.nn.Linear(256, 192, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(g.standard_normal((192, 256)) * 0.05, dev, torch.bfloat16))
    scale = to_dev(g.uniform(0.5, 2.0, size=(256,)), dev)
    mod = FakeQuantLinear(lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64,
                          symmetric=True, clip_ratio=1.0, online_hadamard=block is not None,
                          online_hadamard_block_size=block, input_scale=scale)
    w_ref = OQ.fake_quantize_hif4(lin.weight.detach().float().cpu().numpy(), HIF4_SCALE_LEVELS, dtype="bfloat16")
    assert np.array_equal(mod.weight.float().cpu().numpy(), w_ref)
    x = to_dev(g.standard_normal((4, 33, 256)), dev, torch.bfloat16)
    # the reference's steps (quantization.py:204-276) with this library's standalone ops
    ref_x = x * scale.to(torch.bfloat16)
    if block is not None:
        ref_x = _ops.hadamard_rows(ref_x.float(), block, out_dtype=torch.bfloat16)
    ref_x = fake_quantize(ref_x, quant_format="hif4", bits=4, group_size=64)
    expected = torch.nn.functional.linear(ref_x, mod.weight, mod.bias)
    got = mod(x)
    assert torch.equal(got, expected)
    assert HIF4_ACT_SCALE_LEVELS in ("123", "12", "13")


def test_fake_quant_linear_unsupported_options_raise(dev):
    from faquant_amd.quantization import FakeQuantLinear

    lin = torch.nn.Linear(64, 64).to(dev)
    common = dict(quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64, symmetric=True,
                  clip_ratio=1.0)
    with pytest.raises(ValueError):
        FakeQuantLinear(lin, **{**common, "weight_group_size": 32})
    with pytest.raises(ValueError, match="signs and permutation"):
        FakeQuantLinear(lin, **common, input_rotation_signs=torch.ones(64, dtype=torch.int8))
    with pytest.raises(ValueError, match="permutation of the input features"):
        FakeQuantLinear(lin, **common, input_rotation_signs=torch.ones(64, dtype=torch.int8),
                        input_rotation_permutation=torch.zeros(64, dtype=torch.long))


# ---------------------------------------------------------------- the full activation path

_TORCH_DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _prep_on_device(x, dtype, dev, levels, kw):
    """oracle.linear keyword arguments -> _ops.act_prep_rows on the device."""
    from faquant_amd import _ops

    def t(a, dt=torch.float32):
        return None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt)

    return _ops.act_prep_rows(
        to_dev(x, dev, _TORCH_DT[dtype]), levels=levels, col_scale=t(kw.get("input_scale")),
        rot_signs=t(kw.get("rot_signs"), torch.int8), rot_perm=t(kw.get("rot_perm"), torch.int64),
        rot_block=kw.get("rot_block"), act_min=kw.get("act_min"), act_max=kw.get("act_max"),
        compand=t(kw.get("compand")), hadamard=kw.get("hadamard", 0),
        hadamard_generalized=kw.get("hadamard_generalized", False),
    )


def _same(got, ref):
    """Bitwise equality of fp32 arrays (so -0 differs from +0), any NaN matching any NaN."""
    g, r = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    if g.shape != r.shape:
        return False
    return bool(np.all((g.view(np.uint32) == r.view(np.uint32)) | (np.isnan(g) & np.isnan(r))))


def test_act_prep_rows_matches_reference_fixtures(dev):
    """The reference's FakeQuantLinear wrote these activations (tests/golden/linear_act.npz)."""
    from oracle import linear as OL
    from tests.linear_cases import golden_cases

    for name, c in sorted(golden_cases().items()):
        print(f"[act_prep golden] {name}", flush=True)
        got = _prep_on_device(c["x"], c["dtype"], dev, c["levels"], c["kw"]).float().cpu().numpy()
        assert _same(got, c["y"]), name
        assert _same(got, OL.fake_quant_linear_input(c["x"], c["dtype"], levels=c["levels"], **c["kw"]))


def _random_prep_case(seed, cols, dtype, *, rot, rot_block, clamp, comp, hadamard, scale):
    from tests.linear_cases import compand_scale

    g = OI.rng(seed)
    rows = 13
    x = g.standard_normal((rows, cols)) * np.exp(g.standard_normal((rows, 1)))
    x[g.integers(0, rows, 5), g.integers(0, cols, 5)] *= 30.0
    x[2, 64:192] = 0.0
    x = OQ.bf16_round(x) if dtype == "bfloat16" else (
        x.astype(np.float16).astype(np.float32) if dtype == "float16" else x.astype(np.float32))
    kw = {"hadamard": hadamard}
    if scale:
        kw["input_scale"] = g.uniform(0.3, 3.0, cols).astype(np.float32)
    if rot:
        kw["rot_signs"] = g.choice(np.array([-1, 1], np.int8), cols)
        kw["rot_perm"] = g.permutation(cols)
        kw["rot_block"] = rot_block
    if clamp:
        kw["act_min"], kw["act_max"] = -float(g.uniform(0.5, 4)), float(g.uniform(0.5, 4))
    if comp:
        kw["compand"] = compand_scale(g.uniform(-3, 3, cols // 64).astype(np.float32), cols, dtype)
    return x, kw


PREP_CONFIGS = {
    # name: (cols, rot, rot_block, clamp, comp, hadamard, scale)
    "rot_perm_only": (1024, True, None, False, False, 0, False),
    "rot64_clamp": (1024, True, 64, True, False, 0, True),
    "rot1024_all": (2048, True, 1024, True, True, 128, True),
    "norot_clamp_comp_h512": (1536, False, None, True, True, 512, False),
    "rot4096_h4096": (4096, True, 4096, False, True, 4096, True),
    "qwen8b_down_12288": (12288, True, 1024, True, True, 0, False),
    "max_16384_norot": (16384, False, None, True, False, 1024, True),
    "qwen32b_down_25600": (25600, True, 1024, True, True, 0, False),
    "max_32768": (32768, True, 2048, True, True, 4096, True),
}


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("levels", ["123", "12", "13"])
@pytest.mark.parametrize("name", sorted(PREP_CONFIGS))
def test_act_prep_rows_matches_oracle_bitwise(dev, name, levels, dtype):
    from oracle import linear as OL

    cols, rot, rot_block, clamp, comp, hadamard, scale = PREP_CONFIGS[name]
    x, kw = _random_prep_case(zlib.crc32(f"{name}/{levels}/{dtype}".encode()) & 0xFFFF, cols, dtype, rot=rot, rot_block=rot_block,
                              clamp=clamp, comp=comp, hadamard=hadamard, scale=scale)
    print(f"[act_prep] {name} levels={levels} {dtype} cols={cols}", flush=True)
    got = _prep_on_device(x, dtype, dev, levels, kw).float().cpu().numpy()
    ref = OL.fake_quant_linear_input(x, dtype, levels=levels, **kw)
    assert _same(got, ref)


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
@pytest.mark.parametrize("cols", [192, 768, 3072, 12288, 1024])
def test_act_prep_rows_generalized_hadamard_matches_oracle(dev, cols, dtype):
    """The online transform without a block size: generalized_hadamard_transform of the row
    (12 * 2^k, or a power of two), alone and after the rotation, clamp and companding."""
    from oracle import linear as OL

    for extras in (False, True):
        x, kw = _random_prep_case(cols + extras, cols, dtype, rot=extras, rot_block=64 if extras else None,
                                  clamp=extras, comp=extras, hadamard=0, scale=extras)
        kw["hadamard_generalized"] = True
        print(f"[act_prep generalized] cols={cols} {dtype} extras={extras}", flush=True)
        got = _prep_on_device(x, dtype, dev, "123", kw).float().cpu().numpy()
        assert _same(got, OL.fake_quant_linear_input(x, dtype, levels="123", **kw))
    with pytest.raises(ValueError, match="unsupported generalized Hadamard dimension"):  # 320 = 5 * 64
        _prep_on_device(np.ones((2, 320), np.float32), dtype, dev, "123", {"hadamard_generalized": True})


@pytest.mark.filterwarnings("ignore::RuntimeWarning")  # NaN and infinite inputs on purpose
def test_act_prep_rows_nan_and_no_quantizer(dev):
    from oracle import linear as OL

    x, kw = _random_prep_case(77, 512, "bfloat16", rot=False, rot_block=None, clamp=True, comp=True,
                              hadamard=0, scale=False)
    x[1, 7] = np.nan  # the clamp keeps NaN; its quantization group turns NaN
    for levels in ("123", None):
        got = _prep_on_device(x, "bfloat16", dev, levels, kw).float().cpu().numpy()
        assert _same(got, OL.fake_quant_linear_input(x, "bfloat16", levels=levels, **kw))
        assert np.isnan(got[1, 7])
    # leading dimensions, and rows that need two rounds of 8-value lanes per workgroup
    x, kw = _random_prep_case(78, 4096, "bfloat16", rot=True, rot_block=256, clamp=False, comp=False,
                              hadamard=0, scale=False)
    got = _prep_on_device(x, "bfloat16", dev, "123", kw)
    x3 = to_dev(x, dev, torch.bfloat16).reshape(13, 1, 4096)
    from faquant_amd import _ops

    got3 = _ops.act_prep_rows(x3, levels="123", rot_signs=torch.from_numpy(kw["rot_signs"]).to(dev),
                              rot_perm=torch.from_numpy(kw["rot_perm"]).to(dev), rot_block=256)
    assert got3.shape == (13, 1, 4096) and torch.equal(got3.reshape(13, 4096), got)


@pytest.mark.filterwarnings("ignore::RuntimeWarning")  # NaN and infinite inputs on purpose
def test_act_prep_rows_edges(dev):
    """One 64-feature row, a single row, many rows, fp16 infinities through the clamp,
    misaligned option vectors (realigned on the host) and an empty batch."""
    from oracle import linear as OL
    from faquant_amd import _ops

    for cols, rows, dtype in ((64, 1, "bfloat16"), (64, 5000, "float16"), (2048, 1, "float32")):
        x, kw = _random_prep_case(cols + rows, cols, dtype, rot=True, rot_block=min(cols, 64), clamp=True, comp=True,
                                  hadamard=32, scale=True)
        x = np.resize(x, (rows, cols)).astype(np.float32)
        if dtype == "float16":
            x[0, :3] = [np.inf, -np.inf, 70000.0]  # clamped to the bounds (70000 is inf in fp16)
        print(f"[act_prep edge] cols={cols} rows={rows} {dtype}", flush=True)
        got = _prep_on_device(x, dtype, dev, "123", kw).float().cpu().numpy()
        assert _same(got, OL.fake_quant_linear_input(x if dtype != "float16" else x.astype(np.float16).astype(np.float32),
                                                     dtype, levels="123", **kw))
    # option vectors at an offset that is not a multiple of 16 bytes
    x, kw = _random_prep_case(9, 512, "bfloat16", rot=False, rot_block=None, clamp=False, comp=True,
                              hadamard=0, scale=True)
    scale = torch.zeros(513, device=dev)
    scale[1:] = torch.from_numpy(kw["input_scale"]).to(dev)
    comp = torch.zeros(514, device=dev)
    comp[2:] = torch.from_numpy(kw["compand"]).to(dev)
    got = _ops.act_prep_rows(to_dev(x, dev, torch.bfloat16), levels="123", col_scale=scale[1:], compand=comp[2:])
    assert _same(got.float().cpu().numpy(), OL.fake_quant_linear_input(x, "bfloat16", levels="123", **kw))
    empty = _ops.act_prep_rows(torch.empty((0, 512), device=dev, dtype=torch.bfloat16), levels="123",
                               compand=comp[2:])
    assert empty.shape == (0, 512)
    assert _ops.act_qdq_rows(torch.empty((0, 3, 512), device=dev, dtype=torch.bfloat16), levels="123").shape == (0, 3, 512)


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_act_prep_rows_streams_many_rows(dev, dtype):
    """More rows than workgroups (each workgroup streams rows, the next one's load in flight),
    every option on, against the oracle bitwise; then scales outside the product form's
    proven range in a few columns (bf16: subnormal; fp16: 14 and 40), whose waves divide."""
    from oracle import linear as OL

    for cols, rows in ((4096, 1800), (1024, 5000), (12288, 600)):
        x, kw = _random_prep_case(cols ^ rows, cols, dtype, rot=True, rot_block=1024, clamp=True, comp=True,
                                  hadamard=0, scale=True)
        x = np.resize(x, (rows, cols)).astype(np.float32)
        x[::7] *= np.float32(1.5)
        x = OQ.bf16_round(x) if dtype == "bfloat16" else (
            x.astype(np.float16).astype(np.float32) if dtype == "float16" else x)
        print(f"[act_prep stream] cols={cols} rows={rows} {dtype}", flush=True)
        got = _prep_on_device(x, dtype, dev, "123", kw).float().cpu().numpy()
        assert _same(got, OL.fake_quant_linear_input(x, dtype, levels="123", **kw))
        if dtype != "float32" and cols == 4096:
            comp = kw["compand"].copy()
            comp[[5, 700, 3001]] = np.float32(2.0 ** -130) if dtype == "bfloat16" else np.float32([14.0, 40.0, 14.0])
            kw2 = dict(kw, compand=comp)
            print(f"[act_prep stream] divided columns {dtype}", flush=True)
            got = _prep_on_device(x, dtype, dev, "123", kw2).float().cpu().numpy()
            assert _same(got, OL.fake_quant_linear_input(x, dtype, levels="123", **kw2))


def test_compand_reciprocals_and_both_quotient_forms(dev):
    """faq_act_compand_rcp: fp32(1 / c) where the product form is exact for the dtype (bf16:
    normal scales; fp16: |c| < 8), 0 elsewhere and for fp32; and the activation path gives the
    same bits with the reciprocals (product form) and without them (every column divides)."""
    from oracle import linear as OL
    from faquant_amd import _ops

    c = np.float32([0.125, 0.5, 1.0, 3.0, 7.99, 8.0, 14.0, 2.0 ** -130, 1e30, -2.5, 0.0, np.inf] + [1.5] * 4)
    for dtype, keep in (("bfloat16", lambda a: (np.abs(a) >= 2.0 ** -126) & (a != 0)),
                        ("float16", lambda a: np.abs(a) < 8.0), ("float32", lambda a: np.zeros(a.shape, bool))):
        got = _ops.act_compand_rcp(to_dev(c, dev), _TORCH_DT[dtype]).cpu().numpy()
        with np.errstate(divide="ignore", over="ignore"):
            want = np.where(keep(c), np.float32(1.0) / c, np.float32(0.0)).astype(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), dtype
    for dtype in ("bfloat16", "float16"):
        x, kw = _random_prep_case(77, 2048, dtype, rot=True, rot_block=1024, clamp=True, comp=True, hadamard=0,
                                  scale=False)
        x = np.resize(x, (300, 2048)).astype(np.float32)
        xt = to_dev(x, dev, _TORCH_DT[dtype])
        comp = to_dev(kw["compand"], dev)
        args = dict(levels="123", rot_signs=to_dev(kw["rot_signs"], dev, torch.int8),
                    rot_perm=to_dev(kw["rot_perm"], dev, torch.int32), rot_block=1024, act_min=kw["act_min"],
                    act_max=kw["act_max"], compand=comp)
        prod = _ops.act_prep_rows(xt, **args, compand_rcp=_ops.act_compand_rcp(comp, _TORCH_DT[dtype]))
        div = _ops.act_prep_rows(xt, **args, compand_rcp=torch.zeros_like(comp))
        print(f"[compand forms] {dtype}", flush=True)
        ref = OL.fake_quant_linear_input(x, dtype, levels="123", **kw)
        pn, dn = prod.float().cpu().numpy(), div.float().cpu().numpy()
        bad = np.argwhere(pn.view(np.uint32) != dn.view(np.uint32))
        for rr, cc in bad[:8]:
            print(f"  row {rr} col {cc}: product {pn[rr, cc]!r} division {dn[rr, cc]!r} oracle {ref[rr, cc]!r} "
                  f"scale {kw['compand'][cc]!r}", flush=True)
        print(f"  {len(bad)} differ; product==oracle {_same(pn, ref)} division==oracle {_same(dn, ref)}", flush=True)
        assert torch.equal(prod.view(torch.int16), div.view(torch.int16))
        assert _same(pn, ref)


def test_fake_quant_linear_generalized_online_hadamard(dev):
    """online_hadamard without a block size (Qwen3-8B down_proj has 12288 = 12 * 1024 input
    features): the module's activation equals the oracle's generalized transform path."""
    from oracle import linear as OL
    from faquant_amd.hif4 import HIF4_ACT_SCALE_LEVELS
    from faquant_amd.quantization import FakeQuantLinear

    g = OI.rng(33)
    for n in (768, 1024):
        lin = torch.nn.Linear(n, 64, bias=False).to(dev, torch.bfloat16)
        mod = FakeQuantLinear(lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64,
                              symmetric=True, clip_ratio=1.0, online_hadamard=True)
        x = OQ.bf16_round(g.standard_normal((9, n)).astype(np.float32))
        act = OL.fake_quant_linear_input(x, "bfloat16", levels=HIF4_ACT_SCALE_LEVELS, hadamard_generalized=True)
        expected = torch.nn.functional.linear(to_dev(act, dev, torch.bfloat16), mod.weight, mod.bias)
        assert torch.equal(mod(to_dev(x, dev, torch.bfloat16)), expected)


def test_fake_quant_linear_full_path_equals_reference_composition(dev):
    """FakeQuantLinear with every option of the activation path against the oracle's
    activation and F.linear on the same HiF4 weight (quantization.py:199-276)."""
    from oracle import linear as OL
    from faquant_amd.hif4 import HIF4_ACT_SCALE_LEVELS
    from faquant_amd.quantization import FakeQuantLinear

    g = OI.rng(31)
    n, m = 1024, 384
    lin = torch.nn.Linear(n, m, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(g.standard_normal((m, n)) * 0.03, dev, torch.bfloat16))
    signs = g.choice(np.array([-1, 1], np.int8), n)
    perm = g.permutation(n)
    scale = g.uniform(0.5, 2.0, n).astype(np.float32)
    log_scale = g.uniform(-2.5, 2.5, n // 64).astype(np.float32)
    mod = FakeQuantLinear(
        lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64, symmetric=True,
        clip_ratio=1.0, online_hadamard=True, online_hadamard_block_size=128, input_scale=to_dev(scale, dev),
        input_rotation_signs=torch.from_numpy(signs).to(dev), input_rotation_permutation=torch.from_numpy(perm).to(dev),
        input_rotation_block_size=256, activation_min=-2.5, activation_max=3.25,
        activation_compand_log_scale=to_dev(log_scale, dev),
    )
    x = OQ.bf16_round(g.standard_normal((3, 21, n)).astype(np.float32) * 1.7)
    got = mod(to_dev(x, dev, torch.bfloat16))
    # the companding scale as the module computes it, on the device (exp there)
    comp = torch.from_numpy(log_scale).to(dev).repeat_interleave(64).clamp(-2.079, 2.079).exp().to(torch.bfloat16)
    act = OL.fake_quant_linear_input(
        x.reshape(-1, n), "bfloat16", levels=HIF4_ACT_SCALE_LEVELS, input_scale=scale, rot_signs=signs, rot_perm=perm,
        rot_block=256, act_min=-2.5, act_max=3.25, compand=comp.float().cpu().numpy(), hadamard=128,
    )
    expected = torch.nn.functional.linear(to_dev(act, dev, torch.bfloat16), mod.weight, mod.bias)
    assert torch.equal(got.reshape(-1, m), expected)
    # the module caches the kernel's vector forms: an in-place change of a buffer is seen
    with torch.no_grad():
        mod.activation_max.fill_(1.5)
        mod.activation_compand_log_scale.mul_(0.5)
    comp = (torch.from_numpy(log_scale).to(dev) * 0.5).repeat_interleave(64).clamp(-2.079, 2.079).exp()
    comp = comp.to(torch.bfloat16)
    act = OL.fake_quant_linear_input(
        x.reshape(-1, n), "bfloat16", levels=HIF4_ACT_SCALE_LEVELS, input_scale=scale, rot_signs=signs, rot_perm=perm,
        rot_block=256, act_min=-2.5, act_max=1.5, compand=comp.float().cpu().numpy(), hadamard=128,
    )
    expected = torch.nn.functional.linear(to_dev(act, dev, torch.bfloat16), mod.weight, mod.bias)
    assert torch.equal(mod(to_dev(x, dev, torch.bfloat16)).reshape(-1, m), expected)
    # and so is a replaced buffer
    mod.activation_max = torch.tensor(2.0, device=dev)
    act = OL.fake_quant_linear_input(
        x.reshape(-1, n), "bfloat16", levels=HIF4_ACT_SCALE_LEVELS, input_scale=scale, rot_signs=signs, rot_perm=perm,
        rot_block=256, act_min=-2.5, act_max=2.0, compand=comp.float().cpu().numpy(), hadamard=128,
    )
    expected = torch.nn.functional.linear(to_dev(act, dev, torch.bfloat16), mod.weight, mod.bias)
    assert torch.equal(mod(to_dev(x, dev, torch.bfloat16)).reshape(-1, m), expected)


def test_hif4_linear_equals_quantize_then_linear(dev):
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.wan22_hif4 import HiF4Linear, faquant_qdq

    g = OI.rng(9)
    lin = torch.nn.Linear(320, 128, bias=True).to(dev, torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(to_dev(g.standard_normal((128, 320)) * 0.05, dev, torch.bfloat16))
    qdq = faquant_qdq("123")
    mod = HiF4Linear(lin, weight_qdq=qdq, input_qdq=qdq, device=dev, chunk_elements=320 * 64)
    w = fake_quantize_hif4(lin.weight.detach().float(), levels="123").to(torch.bfloat16)
    assert torch.equal(mod.weight, w)
    np.testing.assert_array_equal(mod.weight.float().cpu().numpy(),
                                  OQ.fake_quantize_hif4(lin.weight.detach().float().cpu().numpy(), "123"))
    seen = []
    mod.collector = lambda m, rows, start: seen.append((rows.clone(), start))
    x = to_dev(g.standard_normal((3, 50, 320)), dev, torch.float32)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod(x)
        want = torch.nn.functional.linear(fake_quantize_hif4(x.reshape(-1, 320), levels="123"), mod.weight, mod.bias)
    assert got.shape == (3, 50, 128)
    assert torch.equal(got.reshape(-1, 128), want)
    # the collector sees every quantized input row once, bit-exact with the oracle's QDQ
    assert len(seen) == 1 and seen[0][1] == 0
    np.testing.assert_array_equal(seen[0][0].cpu().numpy(), OQ.fake_quantize_hif4(x.reshape(-1, 320).cpu().numpy(), "123"))
    # and the product is the fp32 product of the HiF4 operands within bf16 GEMM rounding
    ref = seen[0][0].double() @ mod.weight.double().T + mod.bias.double()
    assert float((got.reshape(-1, 128).double() - ref).abs().max() / ref.abs().max()) < 1e-2
    with pytest.raises(RuntimeError, match="exactly representable"):
        HiF4Linear(lin, weight_qdq=lambda w: w * 1.001, input_qdq=qdq, device=dev)
    with pytest.raises(ValueError, match="HiF4 weight of shape"):
        HiF4Linear(lin, weight_qdq=qdq, input_qdq=qdq, device=dev, weight=torch.zeros(3, 3))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_rotation_dropins_on_the_row_kernel(dev, dtype):
    """rotation.py drop-ins that run on the activation row kernel: block sizes above 512,
    the generalized transform (fp32) and its chunked form (fp32 math, one cast back)."""
    from oracle import hadamard as OH
    from faquant_amd import rotation

    g = OI.rng(44)
    rnd = OQ.bf16_round if dtype == "bfloat16" else (lambda a: np.asarray(a, np.float32))
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float32
    for cols, block in ((2048, 1024), (12288, 4096), (16384, 16384)):
        x = rnd(g.standard_normal((6, cols)).astype(np.float32) * 3)
        got = rotation.chunked_block_hadamard_transform(to_dev(x, dev, tdt), block_size=block)
        assert got.dtype == tdt and _same(got.float().cpu().numpy(), rnd(OH.block_hadamard_transform(x, block)))
    for cols in (768, 12288, 2048):
        x = rnd(g.standard_normal((5, cols)).astype(np.float32))
        got = rotation.chunked_generalized_hadamard_transform(to_dev(x, dev, tdt))
        assert _same(got.float().cpu().numpy(), rnd(OH.generalized_hadamard_transform(x)))
        if dtype == "float32":
            got = rotation.generalized_hadamard_transform(to_dev(x, dev))
            assert _same(got.cpu().numpy(), OH.generalized_hadamard_transform(x))
    if dtype == "float32":
        x = g.standard_normal((3, 4096)).astype(np.float32)
        assert _same(rotation.hadamard_transform(to_dev(x, dev)).cpu().numpy(), OH.hadamard_transform(x))
    with pytest.raises(ValueError, match="unsupported generalized"):
        rotation.generalized_hadamard_transform(torch.zeros((1, 320), device=dev))


def test_output_tensors_are_checked(dev):
    """A caller-provided output of the wrong shape, dtype or layout is refused before any
    launch (the kernels write through its pointer)."""
    from faquant_amd import _ops

    x = torch.zeros((4, 256), device=dev, dtype=torch.bfloat16)
    for bad in (torch.empty((4, 128), device=dev, dtype=torch.bfloat16),
                torch.empty((4, 256), device=dev, dtype=torch.float32),
                torch.empty((256, 4), device=dev, dtype=torch.bfloat16).t()):
        with pytest.raises(ValueError, match="out must"):
            _ops.act_qdq_rows(x, levels="123", out=bad)
        with pytest.raises(ValueError, match="out must"):
            _ops.act_prep_rows(x, levels="123", out=bad)
    q = torch.zeros((1, 2, 8, 128), device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="out must"):
        _ops.operand_prep(q, levels="123", out=torch.empty((1, 2, 4, 128), device=dev, dtype=torch.bfloat16))


def test_attention_wrappers_check_output_extent(dev):
    """attention_fwd / attention_decode refuse an output or K that does not cover the rows
    and keys they would touch."""
    from faquant_amd import _ops

    q = torch.zeros((1, 4, 8, 128), device=dev, dtype=torch.bfloat16)
    k = torch.zeros((1, 2, 256, 128), device=dev, dtype=torch.bfloat16)
    vt = torch.zeros((1, 2, 128, 256), device=dev, dtype=torch.bfloat16)
    kw = dict(causal=True, scale=0.088, quant_p=True, p_levels="123", norm_same=True)
    with pytest.raises(ValueError, match="attention output must be"):
        _ops.attention_fwd(q, k, vt, 256, out=torch.empty((1, 4, 4, 128), device=dev), **kw)
    with pytest.raises(ValueError, match="k must be"):
        _ops.attention_fwd(q, k[:, :, :100], vt, 256, out=torch.empty((1, 4, 8, 128), device=dev), **kw)
    with pytest.raises(ValueError, match="row_den"):
        _ops.attention_fwd(q, k, vt, 256, out=torch.empty((1, 4, 8, 128), device=dev),
                           row_den=torch.empty((1, 4, 4), device=dev), **kw)
    with pytest.raises(ValueError, match="attention output must be"):
        _ops.attention_decode(q[:, :, :1], 256, k=k, v=k, out=torch.empty((1, 4, 2, 128), device=dev), **kw)


def test_companding_scale_is_within_one_ulp_of_the_exact_exponential(dev):
    """The companding scale (quantization.py:228-234) is torch's exp of the clamped log
    scale on the buffer's device, then cast to the activation dtype, as in the reference,
    which also takes exp wherever its buffer lives: its last bit is the device's exp.  Pin it
    to exp itself: for fp32 activations within one fp32 ulp of the correctly rounded
    exponential (float64 exp rounded once), and for bf16 activations within one bf16 ulp of it
    (bitwise away from bf16 rounding ties)."""
    from faquant_amd.quantization import FakeQuantLinear

    g = OI.rng(61)
    n = 4096
    log_scale = g.uniform(-2.5, 2.5, n).astype(np.float32)
    exact = np.exp(np.clip(log_scale, np.float32(-2.079), np.float32(2.079)).astype(np.float64))
    lin = torch.nn.Linear(n, 64, bias=False).to(dev, torch.bfloat16)
    mod = FakeQuantLinear(lin, quant_format="hif4", bits=4, weight_group_size=64, activation_group_size=64,
                          symmetric=True, clip_ratio=1.0, activation_compand_log_scale=to_dev(log_scale, dev))
    for dtype, round_exact in ((torch.float32, lambda a: a.astype(np.float32)),
                               (torch.bfloat16, lambda a: OQ.bf16_round(a.astype(np.float32)))):
        _, compand, _, _ = mod._prep_vectors(torch.zeros(1, n, device=dev, dtype=dtype))
        got = compand.cpu().numpy()
        want = round_exact(exact)
        step = np.spacing(want) if dtype == torch.float32 else np.spacing(want) * 65536.0
        off = np.abs(got.astype(np.float64) - want.astype(np.float64)) / step
        print(f"[compand] {dtype}: {int((off > 0).sum())} of {n} differ from the exact value, max {off.max():.2f} ulp",
              flush=True)
        assert off.max() <= 1.0
