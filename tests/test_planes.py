"""Row-codec planes in a .safetensors file: the reference's stored schema
(docs/qwen-safetensors.md:45-58) and its admission (qwen_weights.py:58-92,
183-195), on the CPU."""

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import oracle
from venturi_amd import Q4RowSplitWeight, Q8RowSplitWeight
from venturi_amd.planes import planes_of, plane_schema, read_planes
from venturi_amd.quantization.layout import row_payload_bytes
from venturi_amd.weights import Q5RowSplitWeight


def _q8(n, k, seed):
    gen = torch.Generator().manual_seed(seed)
    return Q8RowSplitWeight.from_dense((torch.randn(n, k, generator=gen) * 0.02).half())


def _q4(n, k, seed):
    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(-8, 8, (n, k), generator=gen)
    scales = (torch.rand(n, -(-k // 64), generator=gen) * 0.01).half()
    return Q4RowSplitWeight.from_codes(codes, scales)


def _q5(n, k, seed):
    gen = torch.Generator().manual_seed(seed)
    codes = torch.randint(-16, 16, (n, k), generator=gen)
    scales = (torch.rand(n, -(-k // 64), generator=gen) * 0.01).half()
    return Q5RowSplitWeight.from_codes(codes, scales)


@pytest.mark.parametrize("fmt", ["q8_g32_fp16", "q4_g64_fp16", "q5_g64_fp16", "q6_g64_fp16"])
@pytest.mark.parametrize("shape", [(7168, 5120), (5120, 17408), (248320, 5120), (3, 1), (5, 129)])
def test_schema_bytes_match_the_row_payload(fmt, shape):
    # The planes hold exactly the row payload (layout.py:34-39): codes, high bits, scales.
    schema = plane_schema("m", fmt, shape)
    total = sum(int(np.prod(s)) * (2 if d == "float16" else 1) for _, s, d in schema)
    assert total == row_payload_bytes(shape, fmt)
    assert [t for t, _, _ in schema][0] == "m.codes" and schema[-1][0] == "m.scales"
    assert (len(schema) == 3) == (fmt in ("q5_g64_fp16", "q6_g64_fp16"))


@pytest.mark.parametrize("make", [_q8, _q4, _q5])
@pytest.mark.parametrize("k", [1, 136, 300])
def test_round_trip(tmp_path, make, k):
    w = make(9, k, k)
    path = tmp_path / "m.safetensors"
    planes = planes_of("model.layers.0.mlp.down_proj", w)
    planes["unrelated.weight"] = torch.ones(3, dtype=torch.float32)  # other tensors are ignored
    save_file(planes, str(path))
    got = read_planes(path, "model.layers.0.mlp.down_proj", w.format, (9, k))
    assert got.shape == (9, k) and got.padded_k == w.padded_k
    back = got.weight()
    assert type(back) is type(w) and back.in_features == k
    assert torch.equal(back.codes, w.codes)
    assert torch.equal(back.scales.view(torch.int16), w.scales.view(torch.int16))
    if isinstance(w, Q5RowSplitWeight):
        assert torch.equal(back.high, w.high)
    else:
        assert got.high is None


def test_q6_planes_read_without_a_resident_descriptor(tmp_path):
    n, k = 6, 200
    padded = 256
    rng = np.random.default_rng(3)
    codes = rng.integers(-32, 32, size=(n, padded))
    codes[:, k:] = 0
    scales = (rng.random((n, padded // 64)) * 0.02).astype(np.float16)
    c, h, s = oracle.pack_row_codec(codes, scales, 6)
    path = tmp_path / "q6.safetensors"
    save_file({"p.codes": torch.from_numpy(c), "p.high": torch.from_numpy(h), "p.scales": torch.from_numpy(s)},
              str(path))
    got = read_planes(path, "p", "q6_g64_fp16", (n, k))
    assert np.array_equal(got.high.numpy(), h) and np.array_equal(got.codes.numpy(), c)
    with pytest.raises(ValueError, match="no resident-weight descriptor"):
        got.weight()


def _write(tmp_path, planes):
    path = tmp_path / "bad.safetensors"
    save_file(planes, str(path))
    return path


def test_admission_errors(tmp_path):
    w = _q8(4, 100, 1)
    good = planes_of("w", w)
    with pytest.raises(ValueError, match="missing plane: w.scales"):
        read_planes(_write(tmp_path, {"w.codes": good["w.codes"]}), "w", w.format, (4, 100))
    with pytest.raises(ValueError, match="shape/dtype mismatch: w.codes"):
        bad = dict(good, **{"w.codes": good["w.codes"].view(torch.uint8)})
        read_planes(_write(tmp_path, bad), "w", w.format, (4, 100))
    with pytest.raises(ValueError, match="shape/dtype mismatch"):
        read_planes(_write(tmp_path, good), "w", w.format, (4, 200))  # K padded to 256, not 128
    with pytest.raises(ValueError, match="shape/dtype mismatch: w.scales"):
        bad = dict(good, **{"w.scales": good["w.scales"].float()})
        read_planes(_write(tmp_path, bad), "w", w.format, (4, 100))
    codes = good["w.codes"].clone()
    codes[2, 7] = -128
    with pytest.raises(ValueError, match="-128"):
        read_planes(_write(tmp_path, dict(good, **{"w.codes": codes})), "w", w.format, (4, 100))
    for value in (float("nan"), float("inf"), -0.5):
        scales = good["w.scales"].clone()
        scales[1, 0] = value
        with pytest.raises(ValueError, match="finite and nonnegative"):
            read_planes(_write(tmp_path, dict(good, **{"w.scales": scales})), "w", w.format, (4, 100))
    q4 = _q4(4, 100, 2)
    with pytest.raises(ValueError, match="missing plane: w.high"):
        read_planes(_write(tmp_path, planes_of("w", q4)), "w", "q5_g64_fp16", (4, 100))
    with pytest.raises(ValueError, match="not a row-codec format"):
        plane_schema("w", "fp16", (4, 100))
    with pytest.raises(ValueError, match="Q8, Q4 or Q5"):
        planes_of("w", torch.zeros(2))


def test_q4_code_minus_8_is_admitted(tmp_path):
    # Only Q8 forbids a code (-128); Q4's -8 (nibble 0x8) is a stored value.
    codes = torch.full((2, 64), -8, dtype=torch.int64)
    w = Q4RowSplitWeight.from_codes(codes, torch.full((2, 1), 0.5).half())
    got = read_planes(_write(tmp_path, planes_of("q", w)), "q", w.format, (2, 64))
    assert bool((got.codes[:, :32] == 0x88).all())
