"""gkv_decode_layer_planned: the layers of one kind in a decode step keep the
split launch's plan once (GKV_PLAN_KEEP) and reuse it (GKV_PLAN_REUSE).

- Every output bit and every cache byte equals gkv_decode_layer's on the same
  inputs, for the keeping call and for reuses after it: full layers (ranges
  that split sequences, combine) and window layers (whole-sequence ranges,
  sequences of length 0 among them).
- A reuse the workspace does not hold a plan for (a plain call planned on it
  since, or another batch size) plans afresh, gives the same bits and sets
  GKV_DEVERR_PLAN.
- A plan reused after the table changed behind the same pointer reads the
  moved block where the table now points (oracle parity, no error); after a
  length changed, the reuse plans afresh (the plain call's bits, the error
  bit set): the key holds a hash of the lengths.
- Config 5's shape (B=1024, contexts U[1024, 3072], window and full layers
  alternating, one workspace per kind): four layers kept/reused against four
  plain calls, outputs and both pool arrays bit for bit.
"""
import numpy as np
import pytest

from kvcase import DecodeCase
from poolcase import PoolLayers

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("window", [0, 128])
def test_planned_layers_match_plain_layer(gkv, cuda, torch_mod, window):
    torch = torch_mod
    rng = np.random.default_rng(300 + window)
    B = 600
    L = rng.integers(0, 2000 if window == 0 else 300, size=B).astype(np.int32)
    L[:4] = [0, 1, 127, 128]
    print(f"planned window={window} B={B}", flush=True)
    case = DecodeCase(B, 64, 8, L, window=window, scale=0.5, seed=301)
    max_len = int(case.seq_lens.max())
    cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, cuda, cos, sin)
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring)
    nbytes = gkv.workspace_bytes(B, 8, max_len, window, 0)
    ws_plain = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    ws_plan = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    k0, v0 = dev["k"].clone(), dev["v"].clone()

    def restore():
        dev["k"].copy_(k0)
        dev["v"].copy_(v0)

    def run(lens, plan=None, ws=None, n=B):
        out = torch.full((n, case.Hq * 64), float("nan"), dtype=torch.float32, device=cuda)
        err = torch.zeros(1, dtype=torch.int32, device=cuda)
        lens_d = torch.from_numpy(lens[:n].astype(np.int32)).to(cuda)
        qkv = dev["qkv"][:n]
        if plan is None:
            gkv.decode_layer(qkv, lens_d, max_len, view, dev["sinks"], out, dev["cos"],
                             dev["sin"], window=window, workspace=ws_plain, dev_err=err)
        else:
            gkv.decode_layer_planned(qkv, lens_d, max_len, view, dev["sinks"], out, dev["cos"],
                                     dev["sin"], plan, window=window, workspace=ws, dev_err=err)
        torch.cuda.synchronize()
        return _bits(out), int(err.item()), dev["k"].clone(), dev["v"].clone()

    lens0 = case.seq_lens.copy()
    lens0[rng.choice(B, 40, replace=False)] = 0
    for lens in (case.seq_lens, lens0):
        restore()
        out_a, err_a, k_a, v_a = run(lens)
        assert err_a == 0
        for plan in (gkv.PLAN_KEEP, gkv.PLAN_REUSE, gkv.PLAN_REUSE):
            restore()
            out_b, err_b, k_b, v_b = run(lens, plan, ws_plan)
            assert err_b == 0, f"plan {plan}: dev_err {err_b}"
            assert np.array_equal(out_b, out_a), f"plan {plan}: output bits differ"
            assert torch.equal(k_b, k_a) and torch.equal(v_b, v_a), f"plan {plan}: cache differs"

    # a plain call plans afresh on the workspace: the kept plan is gone
    restore()
    run(lens0, gkv.PLAN_KEEP, ws_plan)
    restore()
    gkv.decode_layer(dev["qkv"], torch.from_numpy(lens0).to(cuda), max_len, view,
                     dev["sinks"], torch.empty(B, case.Hq * 64, device=cuda), dev["cos"],
                     dev["sin"], window=window, workspace=ws_plan)
    restore()
    out_c, err_c, k_c, v_c = run(lens0, gkv.PLAN_REUSE, ws_plan)
    assert err_c == gkv.DEVERR_PLAN
    restore()
    out_a, _, k_a, v_a = run(lens0)
    assert np.array_equal(out_c, out_a)
    assert torch.equal(k_c, k_a) and torch.equal(v_c, v_a)

    # a plan kept for B sequences is not taken for B - 7
    restore()
    run(lens0, gkv.PLAN_KEEP, ws_plan)
    restore()
    out_d, err_d, _, _ = run(lens0, gkv.PLAN_REUSE, ws_plan, n=B - 7)
    assert err_d == gkv.DEVERR_PLAN
    restore()
    out_e, err_e, _, _ = run(lens0, n=B - 7)
    assert err_e == 0 and np.array_equal(out_d, out_e)


def test_config5_layers_keep_and_reuse(gkv, cuda, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(51)
    B = 1024
    L = rng.integers(1024, 3072 + 1, size=B).astype(np.int32)
    L[1] = 3072
    print(f"config5 planned B={B}", flush=True)
    P = PoolLayers(torch, gkv, L, n_layers=4, window=128, seed=52)
    try:
        ws = {w: torch.empty(gkv.workspace_bytes(B, 8, P.max_len, w), dtype=torch.uint8,
                             device=cuda) for w in (0, 128)}
        before = [P.snapshot(li) for li in range(4)]
        plain_out, plain_kv = [], []
        for li in range(4):
            view = P.views[li]
            out = torch.full((B, 64 * 64), float("nan"), dtype=torch.float32, device=cuda)
            err = torch.zeros(1, dtype=torch.int32, device=cuda)
            gkv.decode_layer(P.t(P.qkv[li]), P.lens_d, P.max_len, view, P.t(P.sinks[li]), out,
                             P.cos_d, P.sin_d, window=view.ring, workspace=ws[view.ring],
                             dev_err=err)
            torch.cuda.synchronize()
            assert int(err.item()) == 0
            plain_out.append(_bits(out))
            plain_kv.append(P.snapshot(li))
        # restore the caches, then the same four layers keeping and reusing
        for li in range(4):
            view = P.views[li]
            n = view.num_blocks * 8 * 16 * 64
            gkv.hip_memcpy_d2d(view.k, before[li][0].data_ptr(), n * 2)
            gkv.hip_memcpy_d2d(view.v, before[li][1].data_ptr(), n * 2)
        torch.cuda.synchronize()
        del before
        for li in range(4):
            view = P.views[li]
            plan = gkv.PLAN_KEEP if li < 2 else gkv.PLAN_REUSE
            print(f"layer {li} window={view.ring} plan={plan}", flush=True)
            out = torch.full((B, 64 * 64), float("nan"), dtype=torch.float32, device=cuda)
            err = torch.zeros(1, dtype=torch.int32, device=cuda)
            gkv.decode_layer_planned(P.t(P.qkv[li]), P.lens_d, P.max_len, view,
                                     P.t(P.sinks[li]), out, P.cos_d, P.sin_d, plan,
                                     window=view.ring, workspace=ws[view.ring], dev_err=err)
            torch.cuda.synchronize()
            assert int(err.item()) == 0
            assert np.array_equal(_bits(out), plain_out[li]), f"layer {li}: output bits differ"
            k1, v1 = P.snapshot(li)
            assert torch.equal(k1, plain_kv[li][0]), f"layer {li}: K cache bytes differ"
            assert torch.equal(v1, plain_kv[li][1]), f"layer {li}: V cache bytes differ"
            del k1, v1
    finally:
        P.close()


@pytest.mark.parametrize("window", [0, 128])
def test_reuse_sees_changed_table_and_lengths(gkv, cuda, torch_mod, window):
    """A plan kept at one call and reused after the table or the lengths
    changed behind the same pointers: a moved block is read where the table
    now points (oracle parity, no error), a changed length makes the reuse
    plan afresh (the plain call's bits, GKV_DEVERR_PLAN set)."""
    from kvcase import allclose_report
    torch = torch_mod
    rng = np.random.default_rng(310 + window)
    B = 300
    L = rng.integers(1, 1500 if window == 0 else 400, size=B).astype(np.int32)
    print(f"stale reuse window={window} B={B}", flush=True)
    case = DecodeCase(B, 64, 8, L, window=window, scale=0.5, seed=311)
    max_len = int(case.seq_lens.max())
    cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, cuda, cos, sin)
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring)
    nbytes = gkv.workspace_bytes(B, 8, max_len, window, 0)
    ws_plain = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    ws_plan = torch.empty(nbytes, dtype=torch.uint8, device=cuda)
    snap = [dev["k"].clone(), dev["v"].clone()]

    def restore():
        dev["k"].copy_(snap[0])
        dev["v"].copy_(snap[1])

    def run(lens, plan=None):
        out = torch.full((B, case.Hq * 64), float("nan"), dtype=torch.float32, device=cuda)
        err = torch.zeros(1, dtype=torch.int32, device=cuda)
        lens_d.copy_(torch.from_numpy(lens.astype(np.int32)))  # same pointer every call
        if plan is None:
            gkv.decode_layer(dev["qkv"], lens_d, max_len, view, dev["sinks"], out, dev["cos"],
                             dev["sin"], window=window, workspace=ws_plain, dev_err=err)
        else:
            gkv.decode_layer_planned(dev["qkv"], lens_d, max_len, view, dev["sinks"], out,
                                     dev["cos"], dev["sin"], plan, window=window,
                                     workspace=ws_plan, dev_err=err)
        torch.cuda.synchronize()
        return out, int(err.item())

    lens_d = torch.from_numpy(case.seq_lens.astype(np.int32)).to(cuda)
    restore()
    _, err = run(case.seq_lens, gkv.PLAN_KEEP)
    assert err == 0

    # Move two blocks of two long sequences: swap their contents in both pools
    # and their table entries, in place. The logical cache is unchanged.
    tab = case.table
    b1, b2 = (int(x) for x in np.argsort(-case.seq_lens)[:2])
    j1, j2 = 0, (int(case.seq_lens[b2]) - 1) % (window or 1 << 30) // 16
    p1, p2 = int(tab[b1, j1]), int(tab[b2, j2])
    assert p1 != p2 and p1 >= 0 and p2 >= 0
    for arr in (dev["k"], dev["v"], snap[0], snap[1]):
        arr[[p1, p2]] = arr[[p2, p1]]
    dev["table"][b1, j1] = p2
    dev["table"][b2, j2] = p1
    restore()
    out_r, err_r = run(case.seq_lens, gkv.PLAN_REUSE)
    assert err_r == 0, f"dev_err {err_r}"
    bad, worst = allclose_report(out_r.cpu().numpy().reshape(B, -1),
                                 case.oracle_out().reshape(B, -1), 2e-3, 1e-2)
    assert bad == 0, f"reuse after a moved block: {bad} outputs off (max err {worst:.3e})"
    restore()
    out_p, _ = run(case.seq_lens)
    assert np.array_equal(_bits(out_r), _bits(out_p))

    # One length changes behind the same pointer: the reuse plans afresh.
    lens2 = case.seq_lens.copy()
    lens2[b1] -= 1
    restore()
    out_r2, err_r2 = run(lens2, gkv.PLAN_REUSE)
    assert err_r2 == gkv.DEVERR_PLAN
    k_r2, v_r2 = dev["k"].clone(), dev["v"].clone()
    restore()
    out_p2, err_p2 = run(lens2)
    assert err_p2 == 0
    assert np.array_equal(_bits(out_r2), _bits(out_p2))
    assert torch.equal(k_r2, dev["k"]) and torch.equal(v_r2, dev["v"])
