"""Descriptor packing: reference known answers, invariants and the numpy oracle."""

import numpy as np
import pytest
import torch

import oracle
from venturi_amd import Q4RowSplitWeight, Q8RowSplitWeight
from venturi_amd.q4 import decode_q4_fp16, quantize_q4_rtn


@pytest.mark.parametrize("k", [1, 31, 32, 65, 128, 129])
def test_q8_nearest_even_stored_scale_and_padding(k):
    """The reference's known-answer input for the Q8 packer (tests/test_q8_weights.py:18-52:
    11 bf16 rows of N(0, 1) * 0.01 from seed 38, row 0 all zero, row chunks of 3 and of 11),
    checked against the format's definition computed here in float32 / float16 with numpy:
    s = fp16(max|x| / 127) per 32-column group of the zero-padded row, q = rint(x / s) clamped
    to [-127, 127], or 0 where s == 0."""
    src = torch.randn(11, k, generator=torch.Generator().manual_seed(38), dtype=torch.bfloat16) * 0.01
    src[0].zero_()
    before = src.clone()
    chunked = {c: Q8RowSplitWeight.from_dense(src, rows_per_chunk=c) for c in (3, 11)}
    assert torch.equal(src, before), "the packer must not modify its source"
    w = chunked[3]
    assert torch.equal(chunked[11].codes, w.codes) and torch.equal(chunked[11].scales, w.scales)
    assert (w.format, w.group_size) == ("q8_g32_fp16", 32)
    assert w.nbytes == w.codes.numel() + 2 * w.scales.numel()

    padded = w.codes.shape[1]
    rows = np.zeros((11, padded), dtype=np.float32)
    rows[:, :k] = src.float().numpy()
    groups = rows.reshape(11, padded // 32, 32)
    s16 = (np.abs(groups).max(axis=2) / np.float32(127)).astype(np.float16)
    s32 = s16.astype(np.float32)[:, :, None]
    safe = np.where(s32 > 0, s32, np.float32(1))
    q = np.where(s32 > 0, np.clip(np.rint(groups / safe), -127, 127), 0).astype(np.int8)
    assert np.array_equal(w.scales.numpy().view(np.uint16), s16.view(np.uint16))
    assert np.array_equal(w.codes.numpy(), q.reshape(11, padded))
    assert int(w.codes.numpy().min()) > -128 and not w.scales[0].any()  # no -128 code; a zero row keeps zero scales
    assert not w.codes[:, k:].any()  # padding columns hold zero codes
    # Reconstruction lies within half a quantization step (plus rounding slack).
    step = np.repeat(s16.astype(np.float64), 32, axis=1)[:, :k]
    err = np.abs(src.double().numpy() - w.dequantize_reference().numpy())
    assert (err <= 0.501 * step + 1e-12).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_q8_pack_matches_numpy_oracle(dtype):
    src = (torch.randn(67, 300, generator=torch.Generator().manual_seed(7)) * 0.02).to(dtype)
    src[3, 40:72] = 0
    w = Q8RowSplitWeight.from_dense(src)
    arr = src.double().numpy() if dtype == torch.float64 else src.float().numpy()
    codes, scales = oracle.q8_pack(arr)
    assert np.array_equal(w.codes.numpy(), codes)
    assert np.array_equal(w.scales.numpy().view(np.uint16), scales.view(np.uint16))


def test_q8_underflow_overflow_nonfinite():
    result = Q8RowSplitWeight.from_dense(torch.full((2, 32), 1e-12))
    assert torch.count_nonzero(result.codes) == torch.count_nonzero(result.scales) == 0
    for value in (float("inf"), float("nan"), 1e12):
        with pytest.raises(ValueError):
            Q8RowSplitWeight.from_dense(torch.full((2, 32), value))
    with pytest.raises(ValueError, match="rows_per_chunk"):
        Q8RowSplitWeight.from_dense(torch.ones(2, 32), rows_per_chunk=0)
    with pytest.raises(TypeError):
        Q8RowSplitWeight.from_dense(
            Q4RowSplitWeight.from_codes(torch.zeros(2, 32, dtype=torch.int8), torch.ones(2, 1, dtype=torch.float16))
        )


@pytest.mark.parametrize("bad", ["codes", "scales", "shape", "noncontiguous"])
def test_q8_descriptor_guards(bad):
    w = Q8RowSplitWeight.from_dense(torch.randn(3, 65))
    kwargs = dict(codes=w.codes, scales=w.scales, in_features=w.in_features)
    if bad == "codes":
        kwargs["codes"] = w.codes.to(torch.uint8)
    elif bad == "scales":
        kwargs["scales"] = w.scales.float()
    elif bad == "shape":
        kwargs["in_features"] = 129
    else:
        kwargs["codes"] = torch.empty(3, 256, dtype=torch.int8)[:, ::2]
    with pytest.raises(ValueError):
        Q8RowSplitWeight(**kwargs)


@pytest.mark.parametrize("k", [1, 63, 64, 65, 127, 128, 129, 4097])
def test_q4_pack_signed_codes_and_tail(k):
    """The reference's storage case (tests/test_q4_weights.py:10-26: codes cycling through all 16
    signed values, group scales (i % 7 + 1) / 8) unpacked here from the layout's definition: column
    2j in the low nibble of byte j, two's complement, rows padded to a multiple of 128 columns."""
    values = (torch.arange(3 * k).reshape(3, k) % 16 - 8).to(torch.int8)
    scales = (torch.arange(3 * ((k + 63) // 64)).reshape(3, -1) % 7 + 1).to(torch.float16) / 8
    weight = Q4RowSplitWeight.from_codes(values, scales)
    assert tuple(weight.codes.shape) == (3, ((k + 127) // 128) * 64)
    raw = weight.codes.numpy()
    nibbles = np.stack((raw & 15, raw >> 4), axis=2).reshape(3, -1)[:, :k].astype(np.int16)
    signed = np.where(nibbles > 7, nibbles - 16, nibbles)
    assert np.array_equal(signed, values.numpy())
    expected = signed * np.repeat(scales.numpy().astype(np.float64), 64, axis=1)[:, :k]
    assert np.array_equal(weight.dequantize_reference().numpy(), expected)
    packed, plane = oracle.q4_pack_codes(values.numpy(), scales.numpy())
    assert np.array_equal(raw, packed) and np.array_equal(weight.scales.numpy(), plane)


def test_q4_known_bytes_and_group_scales():
    # Reference test_q4_weights.py:30-44.
    codes = torch.zeros((1, 64), dtype=torch.uint8)
    codes[0, :3] = torch.tensor([0x10, 0xF8, 0x97], dtype=torch.uint8)
    scales = torch.tensor([[0.5, -2]], dtype=torch.float16)
    weight = Q4RowSplitWeight(codes, scales, 128)
    assert weight.dequantize_reference()[0, :6].tolist() == [0, 0.5, -4, -0.5, 3.5, -3.5]
    assert weight.nbytes == 68


def test_q4_payload_alignment_and_shared_views():
    """One row of 65 columns as a payload (the reference's case, tests/test_q4_weights.py:47-60):
    64 code bytes (65 columns padded to 128) then zeros up to byte 256, then the fp16 scales; the
    descriptor views the payload in place, and any other byte count is refused."""
    codes_plane = np.zeros(256, dtype=np.uint8)
    codes_plane[0] = 0xF8  # column 0: -8, column 1: -1
    scale_plane = np.array([0.5, 2.0], dtype=np.float16).view(np.uint8)
    payload = torch.from_numpy(np.concatenate((codes_plane, scale_plane)))
    weight = Q4RowSplitWeight.from_payload(payload, out_features=1, in_features=65)
    base = payload.data_ptr()
    assert (weight.codes.data_ptr() - base, weight.scales.data_ptr() - base) == (0, 256)
    assert weight.dequantize_reference()[0, :2].tolist() == [-4.0, -0.5]
    for size in (payload.numel() - 1, payload.numel() + 1):
        wrong = torch.zeros(size, dtype=torch.uint8)
        with pytest.raises(ValueError, match="byte count"):
            Q4RowSplitWeight.from_payload(wrong, out_features=1, in_features=65)


@pytest.mark.parametrize("value", [-9, 8])
def test_q4_reject_out_of_range(value):
    with pytest.raises(ValueError, match=r"in \[-8, 7\]"):
        Q4RowSplitWeight.from_codes(torch.tensor([[value]], dtype=torch.int8), torch.ones(1, 1, dtype=torch.float16))


@pytest.mark.parametrize("case", ["dtype", "width", "scales", "stride", "k", "empty"])
def test_q4_reject_bad_storage(case):
    codes = torch.zeros((2, 64), dtype=torch.uint8)
    scales = torch.ones((2, 2), dtype=torch.float16)
    k = 128
    if case == "dtype":
        codes = codes.to(torch.int32)
    if case == "width":
        codes = codes[:, :32].contiguous()
    if case == "scales":
        scales = scales[:, :1].contiguous()
    if case == "stride":
        codes = torch.zeros(2, 128, dtype=torch.uint8)[:, ::2]
    if case == "k":
        k = 0
    if case == "empty":
        codes = codes[:0]
    with pytest.raises(ValueError):
        Q4RowSplitWeight(codes, scales, k)


def test_q4_rtn_ties_tiny_and_saturation():
    # Reference test_flash_next_q4.py:35-48.
    x = torch.zeros(2, 128)
    x[0, :6] = torch.tensor([7.0, 0.5, 1.5, 2.5, -0.5, -1.5])
    x[1, 0] = 1e-10
    q = quantize_q4_rtn(x)
    y = decode_q4_fp16(q)
    assert y[0, :6].tolist() == [7.0, 0.0, 2.0, 2.0, 0.0, -2.0]
    assert not y[1].any() and torch.isfinite(q.scales).all()
    assert q.scales[0, 0] == 1
    assert torch.equal(decode_q4_fp16(Q4RowSplitWeight.from_codes(torch.tensor([[-8, 7, -1, 0]]),
                                                                   torch.tensor([[0.5]], dtype=torch.float16))),
                       torch.tensor([[-4.0, 3.5, -0.5, 0.0]], dtype=torch.float16))


@pytest.mark.parametrize("shape", [(1, 1), (3, 63), (4, 64), (2, 65), (3, 128), (2, 131), (5, 640)])
def test_q4_rtn_matches_oracle_and_scalar_decode(shape):
    torch.manual_seed(223)
    x = torch.randn(shape)
    q = quantize_q4_rtn(x)
    codes, scales = oracle.q4_rtn(x.numpy())
    packed, plane = oracle.q4_pack_codes(codes, scales)
    assert np.array_equal(q.codes.numpy(), packed) and np.array_equal(q.scales.numpy(), plane)
    independent = torch.empty(shape, dtype=torch.float16)
    for row in range(shape[0]):
        for col in range(shape[1]):
            byte = int(q.codes[row, col // 2])
            code = (byte >> (4 * (col % 2))) & 15
            independent[row, col] = (code if code < 8 else code - 16) * float(q.scales[row, col // 64])
    assert torch.equal(decode_q4_fp16(q), independent)
    assert np.array_equal(oracle.q4_decode_fp16(packed, plane, shape[1]), independent.numpy())
    assert not ((q.codes & 15) == 8).any() and not ((q.codes >> 4) == 8).any()
