"""The reference tests' known-answer vectors (tests/golden/known_answers.json)
against this package's codecs and the CPU oracle (no GPU)."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from venturi_amd import Q4RowSplitWeight, Q8RowSplitWeight, decode_q4_fp16, quantize_q4_rtn

GOLDEN = json.loads((Path(__file__).parent / "golden" / "known_answers.json").read_text())


def test_q4_known_bytes():
    g = GOLDEN["q4_known_bytes"]
    codes = torch.zeros(g["codes_shape"], dtype=torch.uint8)
    codes[0, :3] = torch.tensor(g["codes_row0_first_bytes"], dtype=torch.uint8)
    scales = torch.tensor(g["scales"], dtype=torch.float16)
    w = Q4RowSplitWeight(codes, scales, g["in_features"])
    n = len(g["expected_first_values"])
    assert w.dequantize_reference()[0, :n].tolist() == g["expected_first_values"]
    assert w.nbytes == g["expected_nbytes"]
    assert oracle.q4_decode(codes.numpy(), scales.numpy(), g["in_features"]).view(np.float16)[0, :n].tolist() == g[
        "expected_first_values"
    ]


def test_q4_payload_view():
    g = GOLDEN["q4_payload_view"]
    payload = torch.zeros(g["payload_bytes"], dtype=torch.uint8)
    payload[0] = g["byte0"]
    payload[256:].view(torch.float16).copy_(torch.tensor(g["scales_at_256"], dtype=torch.float16))
    w = Q4RowSplitWeight.from_payload(payload, out_features=g["out_features"], in_features=g["in_features"])
    assert w.codes.data_ptr() == payload.data_ptr() and w.scales.data_ptr() == payload.data_ptr() + 256
    assert w.dequantize_reference()[0, :2].tolist() == g["expected_first_values"]


def test_q4_minus8_decode():
    g = GOLDEN["q4_from_codes_minus8"]
    w = Q4RowSplitWeight.from_codes(torch.tensor(g["codes"]), torch.tensor(g["scales"], dtype=torch.float16))
    assert decode_q4_fp16(w).tolist() == g["expected_fp16"]


def test_q4_rtn_ties():
    g = GOLDEN["q4_rtn_ties"]
    x = torch.zeros(g["rows"], g["cols"])
    x[0, : len(g["row0_first"])] = torch.tensor(g["row0_first"])
    x[1, : len(g["row1_first"])] = torch.tensor(g["row1_first"])
    q = quantize_q4_rtn(x)
    y = decode_q4_fp16(q)
    assert y[0, : len(g["expected_row0_first_fp16"])].tolist() == g["expected_row0_first_fp16"]
    assert float(q.scales[0, 0]) == g["expected_scale_row0_group0"]
    assert (not bool(y[1].any())) == g["expected_row1_all_zero"]


def test_a8_ties():
    g = GOLDEN["a8_ties"]
    x = np.zeros((1, g["k"]), dtype=np.float16)
    x[0, : len(g["x_first"])] = g["x_first"]
    codes, scales = oracle.a8_quantize(x.view(np.uint16), g["passes"])
    assert float(scales.ravel()[0]) == g["expected_scale"]
    assert codes.ravel()[: len(g["expected_codes_first"])].tolist() == g["expected_codes_first"]


def test_q8_underflow_and_rejects():
    g = GOLDEN["q8_underflow"]
    w = Q8RowSplitWeight.from_dense(torch.full(g["shape"], g["value"]))
    assert torch.count_nonzero(w.codes) == 0 and torch.count_nonzero(w.scales) == 0
    codes, scales = oracle.q8_pack(np.full(g["shape"], g["value"], dtype=np.float32))
    assert not codes.any() and not scales.any()
    for value in GOLDEN["q8_rejects"]["values"]:
        with pytest.raises(ValueError):
            Q8RowSplitWeight.from_dense(torch.full((2, 32), float(value)))
