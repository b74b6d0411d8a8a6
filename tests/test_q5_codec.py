"""Q5 codec and the oracle's Q4/Q5/Q6 row decode and W5A16 GEMV (no GPU).

The codec checks are the reference's known answers (tests/test_flash_next_q5.py).
The oracle pins are those answers, a scalar decode written from the documented
bit layout, closed forms and inputs built so that a plausible mistake (wrong
nibble, wrong high bit or byte, missing sign extension, wrong scale group,
wrong lane assignment or order) changes the answer.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from venturi_amd.q5 import CODEC, NativeQ5, decode_q5_fp16, quantize_q5_rtn
from venturi_amd.weights import Q5RowSplitWeight

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())["q5"]


def scalar_decode(q):
    """Per-element decode from the descriptor's documented layout (weights.py:175-190)."""
    n, k = q.out_features, q.in_features
    out = torch.empty(n, k, dtype=torch.float16)
    for row in range(n):
        for col in range(k):
            code = (int(q.codes[row, col // 2]) >> (4 * (col % 2))) & 15
            group, lane = col // 64, col % 64
            hb = (int(q.high[row, group * 8 + lane // 8]) >> (lane % 8)) & 1
            signed = code | (hb << 4)
            signed = signed if signed < 16 else signed - 32
            out[row, col] = signed * float(q.scales[row, group])
    return out


@pytest.mark.parametrize("shape", [(1, 1), (3, 63), (4, 64), (2, 65), (3, 128), (2, 131), (5, 640)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_codec_decode_independent_codes_tail_and_owned(shape, dtype):
    torch.manual_seed(229)
    x = torch.randn(shape).to(dtype)
    before = x.clone()
    q = quantize_q5_rtn(x)
    independent = scalar_decode(q)
    assert torch.equal(decode_q5_fp16(q), independent)
    assert torch.equal(x, before)
    assert q.nbytes == shape[0] * q.padded_k * (0.5 + 1 / 8 + 2 / 64)
    # The C oracle's row decoder (bits = 5) agrees element for element.
    got = oracle.row_decode(q.codes.numpy(), q.high.numpy(), q.scales.numpy(), shape[1], 5)
    assert np.array_equal(got, independent.numpy().view(np.uint16))
    x.zero_()
    assert torch.equal(decode_q5_fp16(q), independent)


def test_full_code_range_endpoints_and_ties():
    torch.manual_seed(7)
    x = torch.randn(4, 128) * 0.317
    q = quantize_q5_rtn(x)
    unsigned = torch.stack((q.codes & 15, q.codes >> 4), -1).reshape(4, 2, 64)
    bytes_ = q.high.view(4, 2, 8)
    bits = (bytes_.unsqueeze(-1).to(torch.int16) >> torch.arange(8, dtype=torch.int16)) & 1
    lanes = unsigned.to(torch.int16) | (bits.reshape(4, 2, 64) << 4)
    assert lanes.min() >= 0 and lanes.max() <= 31
    # RTN with scale max|w|/15 saturates at +15/-16; +16 is unreachable.
    expected = (x.reshape(4, 2, 64) / q.scales.float().unsqueeze(-1)).round().clamp(-16, 15)
    assert torch.equal(expected.to(torch.int16) & 31, lanes.to(torch.int16))
    g = GOLDEN["from_codes"]
    q2 = Q5RowSplitWeight.from_codes(torch.tensor(g["codes"]), torch.tensor(g["scales"], dtype=torch.float16))
    assert decode_q5_fp16(q2).tolist() == g["expected"]
    assert oracle.row_decode(q2.codes.numpy(), q2.high.numpy(), q2.scales.numpy(), 8, 5).view(
        np.float16).tolist() == g["expected"]


def test_from_codes_roundtrip_all_thirty_two_codes():
    codes = torch.arange(-16, 16, dtype=torch.int16).reshape(1, 32)
    q = Q5RowSplitWeight.from_codes(codes, torch.tensor([[0.25]], dtype=torch.float16))
    want = [c * 0.25 for c in range(-16, 16)]
    assert decode_q5_fp16(q).tolist() == [want]
    assert q.dequantize_reference().flatten().tolist() == want
    assert oracle.row_decode(q.codes.numpy(), q.high.numpy(), q.scales.numpy(), 32, 5).view(
        np.float16).tolist() == [want]


def test_zero_group_and_saturation_scale():
    g = GOLDEN["saturation"]
    x = torch.zeros(2, 128)
    x[0, :6] = torch.tensor(g["row0"])
    x[1, 0] = 1e-10
    q = quantize_q5_rtn(x)
    y = decode_q5_fp16(q)
    assert y[0, :6].tolist() == g["expected_row0"]
    assert not y[1].any() and torch.isfinite(q.scales).all()
    assert q.scales[0, 0] == g["scale"]


@pytest.mark.parametrize("bad", [torch.tensor([[float("nan")]]), torch.tensor([[float("inf")]]),
                                 torch.tensor([[1e20]]), torch.empty(0, 2), torch.ones(3),
                                 torch.ones(1, 1, dtype=torch.int64)])
def test_quantizer_rejects_invalid_source(bad):
    with pytest.raises(ValueError):
        quantize_q5_rtn(bad)


def test_descriptor_validation_and_admission(tmp_path):
    with pytest.raises(ValueError):
        Q5RowSplitWeight(torch.zeros(1, 64, dtype=torch.uint8), torch.zeros(1, 16, dtype=torch.uint8),
                         torch.zeros(1, 2, dtype=torch.float32), 64)
    with pytest.raises(ValueError):
        Q5RowSplitWeight.from_codes(torch.tensor([[16]]), torch.tensor([[0.5]], dtype=torch.float16))
    with pytest.raises(ValueError):
        Q5RowSplitWeight.from_codes(torch.tensor([[-17]]), torch.tensor([[0.5]], dtype=torch.float16))
    for size in [0, -1, True, 1]:
        with pytest.raises(ValueError):
            quantize_q5_rtn(torch.ones(2, 2), max_elements=size)
    for size in [0, -1, True]:
        with pytest.raises(ValueError):
            NativeQ5(tmp_path / "missing.so", max_output_bytes=size)
    with pytest.raises(FileNotFoundError):
        NativeQ5(tmp_path / "missing.so")
    native = NativeQ5.__new__(NativeQ5)
    native.max_output_bytes = 100000
    for scales in [torch.tensor([[float("nan"), 0]], dtype=torch.float16),
                   torch.tensor([[-1.0, 0]], dtype=torch.float16)]:
        q = Q5RowSplitWeight(torch.zeros(1, 64, dtype=torch.uint8), torch.zeros(1, 16, dtype=torch.uint8), scales, 128)
        with pytest.raises(ValueError):
            native.prepare(q, device="cuda:0")
    with pytest.raises(ValueError):
        native.linear(torch.ones(1, 2, dtype=torch.float16), None)
    assert CODEC == "rtn_symmetric15_g64_fp16_row_split_k128_v1"


def test_from_dense_matches_rtn_rules():
    torch.manual_seed(3)
    w = torch.randn(6, 200) * 0.05
    q = Q5RowSplitWeight.from_dense(w, rows_per_chunk=4)
    scales = (torch.nn.functional.pad(w, (0, 56)).view(6, 4, 64).abs().amax(-1) / 15).half()
    assert torch.equal(q.scales, scales)
    d = q.dequantize_reference()
    bound = scales.double().repeat_interleave(64, 1)[:, :200] / 2
    assert ((d - w.double()).abs() <= bound + 1e-12).all()


# ----------------------------------------------------------- oracle pins


@pytest.mark.parametrize("bits", [4, 5, 6])
@pytest.mark.parametrize("k", [1, 63, 64, 130, 257])
def test_row_decode_every_code_and_group(bits, k):
    # Every code of the range at every lane position, a distinct power-of-two
    # scale per group (so a wrong group index changes the value), and a
    # closed form q * scale that is exact in fp16.
    n, padded = 3, (k + 127) // 128 * 128
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    span = hi - lo + 1
    cols = np.arange(padded)
    codes = np.stack([lo + (cols * 7 + 3 * r) % span for r in range(n)]).astype(np.int64)
    codes[:, k:] = 0
    groups = padded // 64
    scales = np.array([[2.0 ** -(1 + (g + r) % 4) for g in range(groups)] for r in range(n)], dtype=np.float16)
    packed, high, plane = oracle.pack_row_codec(codes, scales, bits)
    got = oracle.row_decode(packed, high, plane, k, bits).view(np.float16)
    want = (codes[:, :k] * scales.astype(np.float64).repeat(64, 1)[:, :k]).astype(np.float16)
    assert np.array_equal(got, want)
    if bits == 4:
        assert np.array_equal(got.view(np.uint16), oracle.q4_decode(packed, plane, k))
    ids = np.array([2, 0, 2], dtype=np.int64)
    assert np.array_equal(oracle.row_decode(packed, high, plane, k, bits, ids).view(np.float16), want[ids])


def test_row_decode_high_plane_bit_order():
    # One set upper bit at a time: column c's upper bits start at bit c*hb of
    # the row's stream (LSB first), so exactly column c becomes negative.
    for bits, c in [(5, 0), (5, 9), (5, 63), (5, 70), (6, 1), (6, 5), (6, 66)]:
        hb = bits - 4
        high = np.zeros((1, 128 * hb // 8), dtype=np.uint8)
        bit = c * hb + hb - 1  # the sign bit of column c
        high[0, bit // 8] |= 1 << (bit % 8)
        codes = np.zeros((1, 64), dtype=np.uint8)
        got = oracle.row_decode(codes, high, np.ones((1, 2), np.float16), 128, bits).view(np.float16)[0]
        want = np.zeros(128)
        want[c] = -(1 << (bits - 1))
        assert np.array_equal(got, want), (bits, c)


def test_q5_linear_impulse_picks_each_weight():
    gen = torch.Generator().manual_seed(5)
    n, k = 3, 130
    codes = torch.randint(-16, 16, (n, k), generator=gen)
    scales = (torch.rand(n, 3, generator=gen) * 0.1).half()
    q = Q5RowSplitWeight.from_codes(codes, scales)
    x = np.eye(k, dtype=np.float16)
    y = oracle.q5_linear(x.view(np.uint16), q.codes.numpy(), q.high.numpy(), q.scales.numpy(), k)
    assert np.array_equal(y.T, decode_q5_fp16(q).numpy().view(np.uint16))


def test_q5_linear_lane_assignment_and_order():
    # flash_next_q5.cu:31-32: lane l owns columns l, l+32, l+64 in order.
    def case(small_col):
        q = Q5RowSplitWeight.from_codes(torch.ones(1, 192, dtype=torch.int8), torch.ones(1, 3, dtype=torch.float16))
        x = np.zeros((1, 192), dtype=np.float16)
        x[0, 0], x[0, 64], x[0, small_col] = 2048, -2048, 2.0**-14
        return oracle.q5_linear(x.view(np.uint16), q.codes.numpy(), q.high.numpy(), q.scales.numpy(), 192)

    assert case(32).view(np.float16)[0, 0] == 0  # (B + small) - B in lane 0
    assert case(1).view(np.float16)[0, 0] == 2.0**-14  # small in lane 1 survives


def test_q5_linear_fp64_bound():
    gen = torch.Generator().manual_seed(17)
    n, k, t = 9, 333, 3
    codes = torch.randint(-16, 16, (n, k), generator=gen)
    scales = (torch.rand(n, 6, generator=gen) * 0.05).half()
    q = Q5RowSplitWeight.from_codes(codes, scales)
    x = torch.randn(t, k, generator=gen).half()
    y = oracle.q5_linear(x.numpy().view(np.uint16), q.codes.numpy(), q.high.numpy(), q.scales.numpy(), k)
    y = y.view(np.float16).astype(np.float64)
    wd = (codes.double() * scales.double().repeat_interleave(64, 1)[:, :k]).numpy().astype(np.float16)
    exact = x.double().numpy() @ wd.astype(np.float64).T
    mag = np.abs(x.double().numpy()) @ np.abs(wd.astype(np.float64)).T
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 2.0**-14))) - 10)
    assert (np.abs(y - exact) <= 0.5 * ulp + k * 2.0**-24 * mag).all()


@pytest.mark.parametrize("bits", [5, 6])
@pytest.mark.parametrize("n", [1, 37])
def test_tiled_copy_layout(bits, n):
    # q5.tile_row_codec's decode copy read back by its documented layout, one
    # weight at a time: nibble j of a word is column c + 2j, nibble 4 + j column
    # c + 2j + 1; the pair (c + 2m, c + 2m + 1) of word jj of high register i
    # sits at bits hb * jj + (0, 8, 4, 12)[m] and 16 above, biased by
    # 2^(bits - 1). Every code of the range, rows past n zero.
    from venturi_amd.q5 import tile_row_codec

    hb = bits - 4
    k, padded = 264, 384
    rng = np.random.default_rng(bits + n)
    codes = rng.integers(-(1 << (bits - 1)), 1 << (bits - 1), size=(n, padded))
    codes[0, :64] = np.arange(-(1 << (bits - 1)), 1 << (bits - 1)).repeat(64 >> (bits - 1))[:64]
    codes[:, k:] = 0
    scales = (rng.random((n, padded // 64)) * 0.02).astype(np.float16)
    packed, high, sc = oracle.pack_row_codec(codes, scales, bits)
    tc, th, ts = tile_row_codec(torch.from_numpy(packed), torch.from_numpy(high), torch.from_numpy(sc), bits)
    tc, th, ts = tc.numpy(), th.numpy(), ts.numpy()
    blocks, chunks = (n + 15) // 16, padded // 128
    assert tc.shape == (blocks, chunks, 4, 16, 16) and th.shape == (blocks, chunks, 4, 16, 4 * hb)
    regs = th.reshape(blocks, chunks, 4, 16, hb, 4).astype(np.uint32)
    regs = regs[..., 0] | (regs[..., 1] << 8) | (regs[..., 2] << 16) | (regs[..., 3] << 24)
    per = 4 // hb
    got = np.zeros((blocks * 16, padded), np.int64)
    for blk in range(blocks):
        for c in range(chunks):
            for q in range(4):
                for r in range(16):
                    word_bytes = tc[blk, c, q, r]
                    for j in range(4):
                        word = int.from_bytes(bytes(word_bytes[4 * j:4 * j + 4]), "little")
                        reg = int(regs[blk, c, q, r, j // per])
                        base = hb * (j % per)
                        for m in range(4):
                            for side in range(2):  # column c + 2m + side
                                nibble = (word >> (4 * (m + 4 * side))) & 15
                                field = (reg >> (base + (0, 8, 4, 12)[m] + 16 * side)) & ((1 << hb) - 1)
                                col = 128 * c + 32 * q + 8 * j + 2 * m + side
                                got[16 * blk + r, col] = (nibble | (field << 4)) - (1 << (bits - 1))
    assert np.array_equal(got[:n], codes)
    # Rows past n hold all-zero bytes (code -2^(bits-1) with scale 0: never stored).
    assert not tc[-1, :, :, (n - 1) % 16 + 1:].any() and not th[-1, :, :, (n - 1) % 16 + 1:].any()
    assert np.array_equal(ts.transpose(0, 2, 1, 3).reshape(blocks * 16, chunks * 2)[:n], sc)
