"""GPU parity of the HiF4 codec, the Hadamard kernels and the operand prologue.

Bar: bit-exact against the oracle (itself bit-exact with the reference, see
test_oracle_*.py) and against the reference's golden vectors.
"""

import numpy as np
import pytest

from oracle import hadamard as OH
from oracle import hif4 as OQ

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(dtype)


def bits(t):
    return t.float().cpu().numpy().view(np.uint32)


LEVELS = ("123", "12", "13")


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_known_answer_vector(dev, dtype):
    from faquant_amd.quantization import fake_quantize

    x = torch.linspace(-17.25, 18.75, 70, dtype=torch.float32)
    tdt = torch.float32 if dtype == "float32" else torch.bfloat16
    got = fake_quantize(x.to(dev).to(tdt), quant_format="hif4", bits=4, group_size=64)
    assert got.dtype == tdt
    expected = OQ.fake_quantize(x.numpy() if dtype == "float32" else OQ.bf16_round(x.numpy()),
                                quant_format="hif4", bits=4, group_size=64, dtype=dtype)
    np.testing.assert_array_equal(bits(got), expected.view(np.uint32))
    assert got.float().cpu()[2].item() == (-17.5 if dtype == "bfloat16" else -15.0)


@pytest.mark.parametrize("levels", LEVELS)
def test_golden_vectors_bit_exact(dev, golden_codec, levels):
    from faquant_amd.hif4 import fake_quantize_hif4, fit_hif4_compact_parameters

    g = golden_codec
    np.testing.assert_array_equal(bits(fake_quantize_hif4(to_dev(g["x"], dev), levels=levels)),
                                  g[f"y_{levels}"].view(np.uint32))
    yb = fake_quantize_hif4(to_dev(g["x_bf16"], dev, torch.bfloat16), levels=levels)
    np.testing.assert_array_equal(bits(yb), g[f"yb_{levels}"].view(np.uint32))
    for w in (70, 100):
        np.testing.assert_array_equal(bits(fake_quantize_hif4(to_dev(g[f"tail{w}"], dev), levels=levels)),
                                      g[f"ytail{w}_{levels}"].view(np.uint32))
    p = fit_hif4_compact_parameters(to_dev(g["x"], dev).reshape(-1, 64), levels=levels)
    np.testing.assert_array_equal(p.scale.reshape(-1).cpu().numpy(), g[f"scale_{levels}"])
    np.testing.assert_array_equal(p.reciprocal.reshape(-1).cpu().numpy(), g[f"rec_{levels}"])
    np.testing.assert_array_equal(p.scale_lv2_exponent.reshape(-1, 8).cpu().numpy(), g[f"lv2_{levels}"])
    np.testing.assert_array_equal(p.scale_lv3_exponent.reshape(-1, 16).cpu().numpy(), g[f"lv3_{levels}"])


@pytest.mark.parametrize("levels", LEVELS)
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_random_tensors_bit_exact(dev, levels, dtype):
    from faquant_amd.hif4 import fake_quantize_hif4

    g = np.random.Generator(np.random.PCG64(7))
    x = (g.standard_t(4.0, size=(257, 384)) * np.exp(g.uniform(-6, 6, size=(257, 1)))).astype(np.float32)
    if dtype == "bfloat16":
        x = OQ.bf16_round(x)
    elif dtype == "float16":
        x = OQ.fp16_round(np.clip(x, -6e4, 6e4))
    tdt = getattr(torch, dtype)
    got = fake_quantize_hif4(to_dev(x, dev, tdt), levels=levels)
    exp = OQ.fake_quantize_hif4(x, levels, dtype)
    np.testing.assert_array_equal(bits(got), exp.view(np.uint32))


def test_exhaustive_scale_sweep(dev):
    """Every positive finite bf16 block maximum, as an all-equal block, through the GPU fit."""
    from faquant_amd.hif4 import fit_hif4_compact_parameters

    maxima = (np.arange(0x0001, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    blocks = np.repeat(maxima[:, None], 64, axis=1)
    for levels in LEVELS:
        p = fit_hif4_compact_parameters(to_dev(blocks, dev), levels=levels)
        s, rec = OQ.e6m2_scale(maxima, levels)
        np.testing.assert_array_equal(p.scale.reshape(-1).cpu().numpy(), s)
        np.testing.assert_array_equal(p.reciprocal.reshape(-1).cpu().numpy(), rec)


def test_special_values(dev):
    from faquant_amd.hif4 import fake_quantize_hif4

    x = np.zeros((4, 64), np.float32)
    x[0] = np.inf  # saturates at the 49152 scale clamp
    x[1, 0] = -np.inf
    x[1, 1:] = 1.0
    x[2, 5] = np.nan  # a NaN makes its whole block NaN, as torch propagates it
    x[3, ::2] = -0.0
    got = fake_quantize_hif4(to_dev(x, dev), levels="123").cpu().numpy()
    assert np.all(got[0] == np.float32(1.75 * 49152 * 4))
    assert got[1, 0] == -np.float32(1.75 * 49152 * 4)
    assert np.all(np.isnan(got[2]))
    assert not np.any(np.signbit(got[3]))  # torch.sign(-0.0) = +0.0


@pytest.mark.parametrize("levels", LEVELS)
def test_packed_encoding_matches_oracle(dev, levels):
    from faquant_amd.hif4 import decode_hif4, encode_hif4, fake_quantize_hif4

    g = np.random.Generator(np.random.PCG64(8))
    x = g.standard_normal((96, 256)).astype(np.float32)
    packed = encode_hif4(to_dev(x, dev), levels=levels)
    ref = OQ.encode(x, levels)
    codes = packed.codes.cpu().numpy()
    nib = np.stack([codes & 15, codes >> 4], axis=-1).reshape(96, 256)
    np.testing.assert_array_equal(nib, ref["codes"])
    np.testing.assert_array_equal(packed.scale_byte.cpu().numpy(), ref["scale_byte"])
    np.testing.assert_array_equal(packed.lv2_bits.cpu().numpy(), ref["lv2_bits"])
    np.testing.assert_array_equal(packed.lv3_bits.cpu().numpy().astype(np.uint16), ref["lv3_bits"])
    dec = decode_hif4(packed)
    np.testing.assert_array_equal(bits(dec), bits(fake_quantize_hif4(to_dev(x, dev), levels=levels)))


def test_packed_storage_round_trip_extremes_and_size(dev):
    """Packed HiF4 (4.5 bits per value) decodes exactly, to fp32 and bf16, over the whole
    E6M2 scale range.  (HiF4 QDQ is not idempotent: the group maximum of a quantized
    group can round to another E6M2 scale, so a cache is packed from the source values.)"""
    from faquant_amd.hif4 import decode_hif4, encode_hif4, fake_quantize_hif4

    g = np.random.Generator(np.random.PCG64(10))
    x = g.standard_normal((3, 5, 512)).astype(np.float32)
    x *= np.exp2(g.integers(-60, 20, size=(3, 5, 8, 1)).astype(np.float32)).repeat(64, axis=-1).reshape(3, 5, 512)
    x[0, 0, :64] = 0.0
    xt = to_dev(x, dev)
    packed = encode_hif4(xt, levels="123")
    nbytes = sum(t.numel() * t.element_size() for t in (packed.codes, packed.scale_byte, packed.lv2_bits,
                                                         packed.lv3_bits))
    assert nbytes * 8 == 4.5 * x.size
    q = fake_quantize_hif4(xt, levels="123")
    np.testing.assert_array_equal(bits(decode_hif4(packed)), bits(q))
    dec16 = decode_hif4(packed, torch.bfloat16)
    assert dec16.dtype == torch.bfloat16 and torch.equal(dec16.float(), q)


def test_qdq_rows_128_matches_oracle(dev):
    from faquant_amd.wan22_attention import qdq_rows_128

    g = np.random.Generator(np.random.PCG64(9))
    x = g.standard_normal((1000, 128)).astype(np.float32)
    np.testing.assert_array_equal(bits(qdq_rows_128(to_dev(x, dev))), OQ.fake_quantize_hif4(x, "123").view(np.uint32))


# ---------------------------------------------------------------- Hadamard

def test_hadamard_golden_bit_exact(dev, golden_hadamard):
    from faquant_amd.rotation import chunked_block_hadamard_transform, hadamard_transform

    g = golden_hadamard
    x = to_dev(g["x"], dev)
    np.testing.assert_array_equal(bits(hadamard_transform(x)), g["h128"].view(np.uint32))
    np.testing.assert_array_equal(bits(hadamard_transform(x.reshape(-1, 64)).reshape(64, 128)), g["h64"].view(np.uint32))
    np.testing.assert_array_equal(bits(chunked_block_hadamard_transform(x, block_size=64)), g["blk64"].view(np.uint32))


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
@pytest.mark.parametrize("n", [8, 64, 128, 512])
def test_hadamard_in_tensor_dtype_matches_reference_goldens(dev, dt, n):
    """hadamard_transform of a bf16 / fp16 tensor runs its butterflies in that dtype
    (rotation.py:14-29): bitwise the reference's output, and the oracle's stage-rounded form
    on random rows."""
    from faquant_amd.rotation import hadamard_transform
    from tests.conftest import load_golden

    g = load_golden("hadamard_native.npz")
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    got = hadamard_transform(to_dev(g[f"x_{dt}_{n}"], dev, tdt))
    assert got.dtype == tdt
    np.testing.assert_array_equal(got.float().cpu().numpy().view(np.uint32), g[f"h_{dt}_{n}"].view(np.uint32))
    rnd = OQ.bf16_round if dt == "bf16" else OQ.fp16_round
    x = rnd(np.random.Generator(np.random.PCG64(n + 7)).standard_normal((777, n)).astype(np.float32) * 3)
    got = hadamard_transform(to_dev(x, dev, tdt)).float().cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), OH.hadamard_transform(x, stage_round=rnd).view(np.uint32))


@pytest.mark.parametrize("n", [2, 8, 16, 32, 64, 128, 256, 512])
def test_hadamard_sizes_bit_exact(dev, n):
    from faquant_amd.rotation import hadamard_transform

    g = np.random.Generator(np.random.PCG64(n))
    x = g.standard_normal((33, max(n, 8) if n >= 8 else 8)).astype(np.float32)
    if n < 8:
        from faquant_amd.rotation import chunked_block_hadamard_transform

        got = chunked_block_hadamard_transform(to_dev(x, dev), block_size=n)
        exp = OH.block_hadamard_transform(x, n)
    else:
        got = hadamard_transform(to_dev(x, dev))
        exp = OH.hadamard_transform(x)
    np.testing.assert_array_equal(bits(got), exp.view(np.uint32))


def test_rotate_heads_matches_oracle(dev):
    from faquant_amd.wan22_attention import rotate_heads

    g = np.random.Generator(np.random.PCG64(3))
    x = OQ.bf16_round(g.standard_normal((2, 50, 3, 128)).astype(np.float32))
    got = rotate_heads(to_dev(x, dev, torch.bfloat16))
    assert got.dtype == torch.bfloat16
    np.testing.assert_array_equal(bits(got), OQ.bf16_round(OH.hadamard_transform(x)).view(np.uint32))


def test_qwen_prologue_golden_bit_exact(dev, golden_hadamard):
    from faquant_amd.qwen3 import post_rope_qk_transform

    g = golden_hadamard
    q = to_dev(g["qwen_q"], dev, torch.bfloat16)
    k = to_dev(g["qwen_k"], dev, torch.bfloat16)
    qr, kr = post_rope_qk_transform(q, k, rotation=True)
    np.testing.assert_array_equal(bits(qr), g["qwen_q_h128"].view(np.uint32))
    np.testing.assert_array_equal(bits(kr), g["qwen_k_h128"].view(np.uint32))
    qb, _ = post_rope_qk_transform(q, k, rotation=True, rotation_block_size=64)
    np.testing.assert_array_equal(bits(qb), g["qwen_q_blk64"].view(np.uint32))
    scale = to_dev(g["smooth_scale"], dev)
    offset = to_dev(g["key_offset"], dev)
    qs, ks = post_rope_qk_transform(q, k, smooth_scale=scale, key_offset=offset, rotation=True)
    np.testing.assert_array_equal(bits(ks), g["qwen_k_offset_smooth_h128"].view(np.uint32))
    np.testing.assert_array_equal(bits(qs), g["qwen_q_smooth_h128"].view(np.uint32))


@pytest.mark.parametrize("levels", LEVELS)
@pytest.mark.parametrize("block", [0, 64, 128])
def test_fused_operand_prologue_bit_exact(dev, levels, block):
    """Hadamard -> bf16 cast -> HiF4 QDQ in one pass equals the oracle's three steps."""
    from faquant_amd import _ops

    g = np.random.Generator(np.random.PCG64(block + 1))
    x = OQ.bf16_round(g.standard_normal((2, 3, 77, 128)).astype(np.float32))
    xt = to_dev(x, dev, torch.bfloat16)
    y, _ = _ops.operand_prep(xt, levels=levels, hadamard=block, round_dtype=torch.bfloat16)
    ref = OH.qk_rotation(x, block_size=block or None, rotate=block != 0, out_round=OQ.bf16_round)
    ref = OQ.fake_quantize_hif4(ref, levels, "bfloat16")
    np.testing.assert_array_equal(bits(y), ref.view(np.uint32))


@pytest.mark.parametrize("src_dtype", ["float32", "bfloat16"])
def test_transposed_value_operand(dev, src_dtype):
    from faquant_amd import _ops

    g = np.random.Generator(np.random.PCG64(4))
    v = g.standard_normal((1, 2, 300, 128)).astype(np.float32)
    if src_dtype == "bfloat16":
        v = OQ.bf16_round(v)
    tdt = getattr(torch, src_dtype)
    # a strided view ([B, L, H, D] storage), as the Wan layout hands it over
    storage = to_dev(np.ascontiguousarray(v.transpose(0, 2, 1, 3)), dev, tdt)
    vt = _ops.operand_prep_vt(storage.transpose(1, 2), levels="123")
    assert vt.shape == (1, 2, 128, 384)
    ref = OQ.fake_quantize_hif4(v, "123", src_dtype)
    got = vt.float().cpu().numpy()
    np.testing.assert_array_equal(got[..., :300].transpose(0, 1, 3, 2).view(np.uint32), ref.view(np.uint32))
    assert np.all(got[..., 300:] == 0)


def test_empty_batches_return_empty(dev):
    """Empty leading dimensions (torch gives the storage a null pointer) pass through the
    quantizer, the Hadamard and the activation prologue as the reference's torch code does."""
    import torch

    from faquant_amd import _ops
    from faquant_amd.hif4 import fake_quantize_hif4
    from faquant_amd.rotation import hadamard_transform

    for dt in (torch.float32, torch.bfloat16):
        x = torch.empty((0, 3, 128), device=dev, dtype=dt)
        assert fake_quantize_hif4(x, levels="123").shape == (0, 3, 128)
        assert _ops.act_qdq_rows(x, levels="123", hadamard=64).shape == (0, 3, 128)
    assert hadamard_transform(torch.empty((0, 64), device=dev)).shape == (0, 64)


def _from_bits(u, dt):
    if dt == "bf16":
        return (u.astype(np.uint32) << 16).view(np.float32)
    return u.view(np.float16).astype(np.float32)


@pytest.mark.parametrize("dt", ["bf16", "fp16"])
def test_in_dtype_transforms_on_the_row_kernel_match_reference_goldens(dev, dt):
    """rotation.hadamard_transform above 512 and rotation.generalized_hadamard_transform on
    bf16 / fp16 tensors run in the tensor's dtype on the activation row kernel (every stage
    and the 12-point mix rounded to it, faq_act_opts.stage_round): bitwise the reference's
    vectors (tests/golden/hadamard_native.npz, keys p*/g*)."""
    from faquant_amd.rotation import generalized_hadamard_transform, hadamard_transform
    from tests.conftest import load_golden

    g = load_golden("hadamard_native.npz")
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    for kind in ("p", "g"):
        for k in sorted(k for k in g if k.startswith(f"{kind}x_{dt}_")):
            n = k.rsplit("_", 1)[1]
            x = to_dev(_from_bits(g[k], dt), dev, tdt)
            fn = hadamard_transform if kind == "p" else generalized_hadamard_transform
            print(f"[in-dtype] {kind} {dt} n={n}", flush=True)
            got = fn(x)
            assert got.dtype == tdt
            np.testing.assert_array_equal(got.float().cpu().numpy().view(np.uint32),
                                          _from_bits(g[f"{kind}h_{dt}_{n}"], dt).view(np.uint32))


@pytest.mark.parametrize("block", [None, 64, 1024])
def test_online_hadamard_linear(dev, block):
    """OnlineHadamardLinear (rotation.py:87-114): the chunked generalized transform of the
    whole row (block None; 12 * 256 = 3072 features) or the per-block transform, cast back
    once, then the wrapped Linear: bitwise the same Linear on the oracle's rotated input."""
    from faquant_amd.rotation import OnlineHadamardLinear

    cols = 3072 if block is None else 2048
    g = np.random.default_rng(70 + (block or 0))
    x = OQ.bf16_round(g.standard_normal((37, cols)).astype(np.float32))
    lin = torch.nn.Linear(cols, 96, bias=True).to(dev).to(torch.bfloat16)
    mod = OnlineHadamardLinear(lin, block_size=block)
    assert mod.faquant_online_hadamard and mod.in_features == cols and mod.out_features == 96
    assert mod.weight is lin.weight and mod.bias is lin.bias
    rot = OH.generalized_hadamard_transform(x) if block is None else OH.block_hadamard_transform(x, block)
    with torch.no_grad():
        got = mod(to_dev(x, dev, torch.bfloat16))
        ref = lin(to_dev(OQ.bf16_round(rot), dev, torch.bfloat16))
    assert torch.equal(got, ref)
