"""Routed-expert Q4 W4A16 MoE on the GPU against the CPU oracle, stage by stage.

* routing: segment offsets equal the per-expert pair counts; every pair has
  one slot inside its expert's segment (exact);
* GEMM outputs (gate, up, y) obey the W4A16 GEMM bound
  |y - exact| <= 0.5 ulp_fp16(exact) + 2^-19 * sum|x w|, so each lies in
  [prev(fp16(exact - d)), next(fp16(exact + d))] with d = 2^-19 * sum|x w|;
* gate/up + SiLU*up (h): inside the oracle's h over the ends and middle of the
  gate and up ranges, widened by 2 fp16 ulps for the fp32 exp inside SiLU
  (the reference's exp is not bit-pinned either); SiLU multiplies a gate ulp
  by about |gate|, so a flat ulp bound does not hold;
* down * score (v), fed the GPU's own h: inside the oracle's v over the ends of
  the y range (v is monotone in y; no widening);
* combine, fed the GPU's own v: bit-exact (ascending expert, fp16 adds);
* end to end vs the oracle: max-abs <= 2e-3 and rel-L2 <= 1e-3.
"""

import numpy as np
import pytest
import torch

import oracle
import oracle.moe as omoe
from helpers import bits
from venturi_amd import Q4RowSplitWeight
from venturi_amd.moe import MoEGeometry, Q4ExpertBank, routed_experts

pytestmark = pytest.mark.gpu


def ulp16(v):
    v = np.abs(v.astype(np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0**-14)))
    return 2.0 ** (e - 10)


def random_q4(n, k, gen, scale):
    codes = torch.randint(-7, 8, (n, k), dtype=torch.int8, generator=gen)
    scales = (torch.rand(n, (k + 63) // 64, generator=gen) * scale + scale / 4).half()
    return Q4RowSplitWeight.from_codes(codes, scales)


def build(backend, device, geometry, seed):
    g = geometry
    gen = torch.Generator().manual_seed(seed)
    experts = [
        (random_q4(2 * g.intermediate_size, g.hidden_size, gen, 0.006), random_q4(g.hidden_size, g.intermediate_size, gen, 0.01))
        for _ in range(g.num_experts)
    ]
    bank = Q4ExpertBank.upload(backend, geometry, experts, device=device)
    gu16 = np.stack([oracle.q4_decode_fp16(e[0].codes.numpy(), e[0].scales.numpy(), g.hidden_size) for e in experts])
    dn16 = np.stack([oracle.q4_decode_fp16(e[1].codes.numpy(), e[1].scales.numpy(), g.intermediate_size) for e in experts])
    return bank, gu16, dn16


def routing(tokens, geometry, seed, duplicates=False):
    gen = torch.Generator().manual_seed(seed)
    ids = torch.stack([torch.randperm(geometry.num_experts, generator=gen)[: geometry.top_k] for _ in range(tokens)])
    if duplicates:
        ids[::3, -1] = ids[::3, 0]
    scores = torch.softmax(torch.randn(tokens, geometry.top_k, generator=gen), -1).half()
    x = torch.randn(tokens, geometry.hidden_size, generator=gen).half()
    return x, ids.to(torch.int64), scores


def fp16_range(x, w):
    """(lower, fp16(exact), upper) fp16 values a GEMM output may take under the W4A16 bound."""
    xd, wd = x.astype(np.float64), w.astype(np.float64)
    exact = xd @ wd.T
    d = 2.0**-19 * (np.abs(xd) @ np.abs(wd).T)
    lo = np.nextafter((exact - d).astype(np.float16), np.float16(-np.inf))
    hi = np.nextafter((exact + d).astype(np.float16), np.float16(np.inf))
    return lo, exact.astype(np.float16), hi


def interval(values):
    stack = np.stack([v.astype(np.float64) for v in values])
    return stack.min(0), stack.max(0)


def run_and_check(backend, device, geometry, tokens, seed, duplicates=False):
    g = geometry
    print(f"case moe E={g.num_experts} H={g.hidden_size} I={g.intermediate_size} K={g.top_k} T={tokens}", flush=True)
    bank, gu16, dn16 = build(backend, device, g, seed)
    x, ids, scores = routing(tokens, g, seed + 1, duplicates)
    plan = bank.prepare(tokens=tokens)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    guard = torch.full((tokens * g.hidden_size + 16,), 47, dtype=torch.float16, device=device)
    out = guard[8:-8].view(tokens, g.hidden_size)
    plan.run(x.to(device), ids.to(device), scores.to(device), out=out, workspace=workspace)
    views = {k: v.cpu().numpy() for k, v in plan.workspace_views(workspace).items()}
    gcpu = guard.cpu()
    assert (gcpu[:8] == 47).all() and (gcpu[-8:] == 47).all()
    ids_np, scores_np, x_np = ids.numpy(), scores.numpy(), x.numpy()
    pairs = tokens * g.top_k

    # Routing.
    seg, slot, slot_token = views["seg"], views["pair_slot"], views["slot_token"]
    assert int(views["status"][0]) == 0
    assert np.array_equal(seg, np.concatenate(([0], np.cumsum(np.bincount(ids_np.ravel(), minlength=g.num_experts)))))
    assert np.array_equal(np.sort(slot.ravel()), np.arange(pairs))
    token_of = np.repeat(np.arange(tokens), g.top_k).reshape(tokens, g.top_k)
    assert np.array_equal(slot_token[slot], token_of)
    assert np.array_equal(views["slot_score"][slot], scores_np)
    assert ((seg[ids_np] <= slot) & (slot < seg[ids_np + 1])).all()

    # Gate/up + SiLU*up, down * score, per expert segment.
    h_gpu, v_gpu = views["h"], views["v"]
    worst_h = worst_v = 0.0
    for e in range(g.num_experts):
        lo, hi = seg[e], seg[e + 1]
        if lo == hi:
            continue
        inter = g.intermediate_size
        rows = x_np[slot_token[lo:hi]]
        gates = fp16_range(rows, gu16[e][:inter])
        ups = fp16_range(rows, gu16[e][inter:])
        hmin, hmax = interval([omoe.fp16_mul(omoe.silu_fp16(a), b) for a in gates for b in ups])
        h = h_gpu[lo:hi].astype(np.float64)
        assert ((h >= hmin - 2 * ulp16(hmin)) & (h <= hmax + 2 * ulp16(hmax))).all()
        h_ref = omoe.fp16_mul(omoe.silu_fp16(gates[1]), ups[1]).astype(np.float64)
        worst_h = max(worst_h, float((np.abs(h - h_ref) / ulp16(h_ref)).max()))
        score = views["slot_score"][lo:hi][:, None]
        ys = fp16_range(h_gpu[lo:hi], dn16[e])
        vmin, vmax = interval([omoe.fp16_mul(a, score) for a in ys])
        v = v_gpu[lo:hi].astype(np.float64)
        assert ((v >= vmin) & (v <= vmax)).all()
        v_ref = omoe.fp16_mul(ys[1], score).astype(np.float64)
        worst_v = max(worst_v, float((np.abs(v - v_ref) / ulp16(v_ref)).max()))

    # Combine (bit-exact given the GPU's v) and end to end.
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint16), omoe.combine(ids_np, slot, v_gpu).view(np.uint16))
    ref = omoe.routed_experts(x_np, ids_np, scores_np, gu16, dn16).astype(np.float64)
    diff = np.abs(got.astype(np.float64) - ref)
    assert diff.max() <= 2e-3
    assert np.linalg.norm(got - ref) <= 1e-3 * max(np.linalg.norm(ref), 1e-12)
    print(f"h worst {worst_h:.2f} ulp, v worst {worst_v:.2f} ulp, out max-abs {diff.max():.3g}", flush=True)
    return plan, bank, (x, ids, scores), out


@pytest.mark.parametrize(
    "geometry,tokens",
    [
        (MoEGeometry(256, 16, 4, 128), 64),
        (MoEGeometry(136, 6, 3, 72), 37),
        (MoEGeometry(512, 8, 2, 200), 1),
        (MoEGeometry(384, 24, 8, 256), 300),
        (MoEGeometry(128, 8, 2, 1032), 40),  # down K of five 256-column chunks, the last one ragged
        # Down's workgroups carry two 256-row tiles of one expert: three tiles leave the
        # last workgroup one (with experts not a multiple of 8, and with three passes).
        (MoEGeometry(640, 10, 3, 96), 70),
        (MoEGeometry(768, 4, 4, 64), 100),
    ],
)
def test_moe_stages(backend, device, geometry, tokens):
    run_and_check(backend, device, geometry, tokens, seed=tokens + geometry.hidden_size)


def test_moe_routing_in_several_batches(backend, device):
    # 1100 tokens x top-8 = 8800 pairs: the routing kernel takes them in three
    # batches of 4096 (ranks of the later ones parked between its passes).
    run_and_check(backend, device, MoEGeometry(64, 16, 8, 32), 1100, seed=21)


def test_moe_repeated_expert_ids(backend, device):
    run_and_check(backend, device, MoEGeometry(128, 8, 4, 64), 30, seed=9, duplicates=True)


def test_moe_config4_and_determinism(backend, device):
    geometry = MoEGeometry(2048, 128, 8, 768)
    plan, bank, (x, ids, scores), out = run_and_check(backend, device, geometry, 512, seed=4)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    again = torch.empty_like(out)
    plan.run(x.to(device), ids.to(device), scores.to(device), out=again, workspace=workspace)
    assert np.array_equal(bits(again), bits(out))
    via_api = routed_experts(x.to(device), ids.to(device), scores.to(device), bank)
    assert np.array_equal(bits(via_api), bits(out))


def test_moe_invalid_ids_give_nan_rows(backend, device):
    geometry = MoEGeometry(128, 8, 2, 64)
    bank, _, _ = build(backend, device, geometry, 3)
    x, ids, scores = routing(4, geometry, 5)
    ids[1, 0] = 8
    ids[2, 1] = -1
    plan = bank.prepare(tokens=4)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    out = torch.empty((4, 128), dtype=torch.float16, device=device)
    plan.run(x.to(device), ids.to(device), scores.to(device), out=out, workspace=workspace)
    views = plan.workspace_views(workspace)
    assert int(views["status"].item()) == 2
    assert int(views["seg"][-1].item()) == 6
    # Tokens with an invalid id get NaN rows; the others equal a run without them.
    rows = out.cpu()
    assert bool(torch.isnan(rows[1]).all()) and bool(torch.isnan(rows[2]).all())
    valid = torch.tensor([0, 3])
    sub = bank.prepare(tokens=2)
    sub_ws = torch.empty(sub.workspace_bytes, dtype=torch.uint8, device=device)
    sub_out = torch.empty((2, 128), dtype=torch.float16, device=device)
    sub.run(x[valid].to(device), ids[valid].to(device), scores[valid].to(device), out=sub_out, workspace=sub_ws)
    assert np.array_equal(bits(sub_out), bits(rows[valid]))
    with pytest.raises(ValueError, match="real expert ids"):
        routed_experts(x.to(device), ids.to(device), scores.to(device), bank)


@pytest.mark.parametrize("geometry,tokens", [(MoEGeometry(512, 16, 4, 256), 64), (MoEGeometry(64, 16, 8, 32), 1100)])
def test_moe_graph_replays(backend, device, geometry, tokens):
    """One plan.run captured in a HIP graph: each replay, on new inputs copied into the captured
    buffers with eager work and synchronisations between, equals an eager run bit for bit
    (in-launch routing at 256 pairs; the separate routing launch at 8800 pairs)."""
    print(f"case moe graph E={geometry.num_experts} H={geometry.hidden_size} T={tokens}", flush=True)
    bank, _, _ = build(backend, device, geometry, 5)
    plan = bank.prepare(tokens=tokens)
    x, ids, scores = (t.to(device) for t in routing(tokens, geometry, 6))
    out = torch.empty((tokens, geometry.hidden_size), dtype=torch.float16, device=device)
    workspace = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
    plan.run(x, ids, scores, out=out, workspace=workspace)  # warm-up outside capture
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.run(x, ids, scores, out=out, workspace=workspace)
    eager = torch.empty_like(out)
    eager_ws = torch.empty_like(workspace)
    for replay in range(3):
        nx, nids, nscores = routing(tokens, geometry, 100 + replay)
        x.copy_(nx.to(device))
        ids.copy_(nids.to(device))
        scores.copy_(nscores.to(device))
        out.fill_(7)
        plan.run(x, ids, scores, out=eager, workspace=eager_ws)  # eager work between replays
        torch.cuda.synchronize(device)
        graph.replay()
        torch.cuda.synchronize(device)
        assert np.array_equal(bits(out), bits(eager)), replay
