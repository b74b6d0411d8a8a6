"""Codec registry geometry and byte accounting (quantization/layout.py, codecs.py)."""

import numpy as np
import pytest
import torch

from venturi_amd.quantization import (
    CODECS,
    EXECUTION_QUALIFIED,
    GFX950,
    ROW_FORMATS,
    codec_for,
    dequantize_planes,
    row_geometry,
    row_payload_bytes,
    validate_reported_plan,
)


def test_formats_and_codecs():
    assert ROW_FORMATS == {"q4_g64_fp16": (4, 64), "q5_g64_fp16": (5, 64), "q6_g64_fp16": (6, 64), "q8_g32_fp16": (8, 32)}
    q8 = codec_for("q8_g32_fp16")
    assert q8.quantized and q8.layout == "row_split_k128_v1" and q8.forbidden_codes == (-128,)
    assert not codec_for("fp16").quantized and codec_for("fp16").dense
    assert set(CODECS) == set(ROW_FORMATS) | {"fp16", "bf16", "fp32"}
    assert EXECUTION_QUALIFIED[GFX950] == {"q8_g32_fp16", "q4_g64_fp16"}
    with pytest.raises(ValueError, match="Unknown weight format"):
        codec_for("q3")


def test_byte_counts_at_baseline_shapes():
    # Config 1: 16 777 216 B codes + 1 048 576 B scales.
    assert row_geometry((4096, 4096), "q8_g32_fp16") == (8, 32, 128, 16777216, 16777216, 17825792)
    assert codec_for("q8_g32_fp16").upload_bytes(4096, 4096) == 17825792
    assert row_payload_bytes((4096, 4096), "q8_g32_fp16") == 17825792
    # Config 2 layer: QKV, o, gate+up, down.
    shapes = [(7168, 5120), (5120, 6144), (34816, 5120), (5120, 17408)]
    assert sum(codec_for("q8_g32_fp16").upload_bytes(n, k) for n, k in shapes) == 356515840
    # Config 4 expert pair (gate_up [1536, 2048] + down [2048, 768]).
    q4 = codec_for("q4_g64_fp16")
    assert q4.upload_bytes(1536, 2048) + q4.upload_bytes(2048, 768) == 2506752
    # Padding: K=65 pads to 128.
    assert codec_for("q8_g32_fp16").encoded_bytes(3, 65) == 3 * (128 + 8)


@pytest.mark.parametrize("fmt,bits", [("q4_g64_fp16", 4), ("q5_g64_fp16", 5), ("q6_g64_fp16", 6)])
def test_all_signed_codes_and_high_bit_positions(fmt, bits):
    """Every signed code of the width, in column order over two 64-column groups (the reference's
    known-answer pattern, tests/test_codec_loading.py:88-113), written into planes built here from
    the layout: low nibbles two per byte, column 2j first; the bits above them as one
    little-endian bit stream of `bits - 4` bits per column; then decoded over 117 columns."""
    values = np.array([(i % (1 << bits)) - (1 << (bits - 1)) for i in range(128)], dtype=np.int64)
    unsigned = values & ((1 << bits) - 1)
    low = (unsigned & 15).reshape(-1, 2)
    codes = torch.from_numpy((low[:, 0] | (low[:, 1] << 4)).astype(np.uint8)[None, :])
    high = None
    if bits > 4:
        hb = bits - 4
        stream = ((unsigned[:, None] >> (4 + np.arange(hb))) & 1).reshape(-1)  # bit b of column c at c * hb + b
        high = torch.from_numpy(np.packbits(stream.astype(np.uint8), bitorder="little")[None, :])
    scales = torch.tensor([[0.125, 0.25]], dtype=torch.float16)
    actual = dequantize_planes(codes, scales, high, (1, 117), fmt)
    group_scale = np.where(np.arange(117) < 64, 0.125, 0.25)
    assert np.array_equal(actual.numpy().astype(np.float64), (values[:117] * group_scale)[None, :])


def test_dequantize_rejects_invalid_planes():
    codes = torch.zeros((1, 128), dtype=torch.int8)
    codes[0, 5] = -128
    with pytest.raises(ValueError, match="Forbidden"):
        dequantize_planes(codes, torch.ones(1, 4, dtype=torch.float16), None, (1, 128), "q8_g32_fp16")
    with pytest.raises(ValueError, match="scale"):
        dequantize_planes(torch.zeros((1, 128), dtype=torch.int8), -torch.ones(1, 4, dtype=torch.float16), None,
                          (1, 128), "q8_g32_fp16")


def test_reported_plan_binding():
    assert validate_reported_plan("q8_g32_fp16", "fp16", GFX950, [8, 32, 0, 0, 0, 0]) == "direct"
    assert validate_reported_plan("q8_g32_fp16", "int8", GFX950, [8, 32, 1, 2, 0, 0]) == "activation-int8"
    assert validate_reported_plan("q4_g64_fp16", "fp16", GFX950, [4, 64, 0, 1, 0, 0]) == "chunked-dense"
    with pytest.raises(RuntimeError):
        validate_reported_plan("q8_g32_fp16", "fp16", GFX950, [8, 32, 1, 0, 0, 0])
    with pytest.raises(ValueError):
        validate_reported_plan("q4_g64_fp16", "fp16", GFX950, [4, 64, 0, 0, 0, 0])


def _spec(**changes):
    from types import SimpleNamespace

    base = dict(target="cuda:0", projection_profile="fp16", linear_implementation="auto", dtype=torch.float16,
                weight_mode="resident", tensor_parallel_device=None, stage_range=None, dequant_resident=False)
    base.update(changes)
    return SimpleNamespace(**base)


def _weights(*formats):
    from types import SimpleNamespace

    return SimpleNamespace(plan=SimpleNamespace(bindings=[SimpleNamespace(format=f) for f in formats]))


def test_linear_contracts_on_gfx950(monkeypatch):
    # quantization/linear.py:16-74 semantics with the gfx950 capability (9, 5).
    from venturi_amd.quantization.linear import describe_linear_contracts, validate_linear_contracts

    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda target: GFX950)
    validate_linear_contracts(_spec(), _weights("q8_g32_fp16", "q4_g64_fp16", "fp16"))
    cases = [
        (_spec(), ("q5_g64_fp16",), "not execution-qualified"),
        (_spec(projection_profile="int8"), ("q8_g32_fp16",), "One-pass int8"),
        (_spec(linear_implementation="fused"), ("q4_g64_fp16",), "Fused model execution"),
        (_spec(dtype=torch.bfloat16), ("q4_g64_fp16",), "row-codec matrices require"),
        (_spec(projection_profile="int8-residual"), ("q4_g64_fp16",), "Residual activation policy"),
        (_spec(linear_implementation="dequant"), ("q8_g32_fp16",), "requires Q4/Q5/Q6 matrices"),
        (_spec(linear_implementation="dequant", stage_range=(0, 4)), ("q8_g32_fp16",), "requires Q4/Q5/Q6"),
        (_spec(dequant_resident=True), ("q4_g64_fp16", "q8_g32_fp16"), "FP16 shadow"),
    ]
    for spec, formats, message in cases:
        with pytest.raises(ValueError, match=message):
            validate_linear_contracts(spec, _weights(*formats))
    monkeypatch.setattr(torch.cuda, "get_device_capability", lambda target: (9, 0))
    with pytest.raises(ValueError, match="Unsupported QuantLinear architecture"):
        validate_linear_contracts(_spec(), _weights("q8_g32_fp16"))
    described = describe_linear_contracts(_weights("q4_g64_fp16", "q8_g32_fp16", "fp16"), "fp16")
    assert described["q4_g64_fp16"]["weight_decode"] == "fp16-rounded-q-times-scale"
    assert described["q8_g32_fp16"]["weight_decode"] == "fp32-scaled-integer-products"
    assert set(described) == {"q4_g64_fp16", "q8_g32_fp16"}
    fused = describe_linear_contracts(_weights("q4_g64_fp16"), "fp16", "fused")
    assert fused["q4_g64_fp16"]["weight_decode"] == "fp32-scaled-integer-products"


@pytest.mark.parametrize("fmt,bits", [("q8_g32_fp16", 8), ("q4_g64_fp16", 4), ("q5_g64_fp16", 5), ("q6_g64_fp16", 6)])
@pytest.mark.parametrize("code_dtype", [torch.uint8, torch.int8])
def test_dequantize_matches_a_per_element_decode(fmt, bits, code_dtype):
    # Random planes against a scalar decode written per column from the layout;
    # the code plane's dtype (int8 or uint8 bytes) must not change the result.
    if bits == 8 and code_dtype == torch.uint8:
        pytest.skip("Q8 codes are int8")
    rng = np.random.default_rng(bits * 7 + (code_dtype == torch.int8))
    rows, cols = 3, 200
    padded = 256
    group = 32 if bits == 8 else 64
    scales = torch.from_numpy(rng.uniform(0, 0.05, (rows, padded // group)).astype(np.float16))
    if bits == 8:
        codes = torch.from_numpy(rng.integers(-127, 128, (rows, padded)).astype(np.int8))
        high = None
    else:
        codes = torch.from_numpy(rng.integers(0, 256, (rows, padded // 2)).astype(np.uint8)).view(code_dtype)
        hb = bits - 4
        high = torch.from_numpy(rng.integers(0, 256, (rows, padded * hb // 8)).astype(np.uint8)) if hb else None
    got = dequantize_planes(codes, scales, high, (rows, cols), fmt).float().numpy()
    body = codes.view(torch.uint8).numpy() if bits < 8 else codes.numpy()
    for r in range(rows):
        for c in range(cols):
            if bits == 8:
                q = int(body[r, c])
            else:
                q = (int(body[r, c // 2]) >> (4 * (c % 2))) & 15
                if bits > 4:
                    hb = bits - 4
                    word = int(high.numpy()[r, (c * hb) // 8])
                    q |= ((word >> ((c * hb) % 8)) & ((1 << hb) - 1)) << 4
                if q >= 1 << (bits - 1):
                    q -= 1 << bits
            expected = np.float16(np.float32(q) * np.float32(scales[r, c // group].item()))
            assert got[r, c] == np.float32(expected), (r, c)
