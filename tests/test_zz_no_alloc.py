"""gkv_decode_layer_noalloc (the decode layer on the library's own scratch, no
allocation) against gkv_decode_layer with a caller workspace: the same cache
bytes and the same output bits, both within the oracle's tolerance. Two calls
in a row on one GPU, the second with a smaller batch (the scratch keeps the
first call's contents), full and window layers."""
import numpy as np
import pytest

from kvcase import DecodeCase, allclose_report, from_pool

pytestmark = pytest.mark.gpu


def _run(case, gkv, torch, dev, noalloc):
    cos, sin = gkv.rope_table(case.cos.shape[0])
    d = case.to_device(torch, dev, cos, sin)
    view = gkv.cache_view(d["k"], d["v"], d["table"], case.Hkv, ring=case.ring)
    max_len = int(case.seq_lens.max())
    out = torch.full((case.B, case.Hq * 64), float("nan"), dtype=torch.float32, device=dev)
    if noalloc:
        gkv.decode_layer_noalloc(d["qkv"], d["seq_lens"], max_len, view, d["sinks"], out,
                                 d["cos"], d["sin"], window=case.window, dev_err=d["err"])
    else:
        ws = torch.empty(gkv.workspace_bytes(case.B, case.Hkv, max_len, case.window),
                         dtype=torch.uint8, device=dev)
        gkv.decode_layer(d["qkv"], d["seq_lens"], max_len, view, d["sinks"], out, d["cos"],
                         d["sin"], window=case.window, workspace=ws, dev_err=d["err"])
    torch.cuda.synchronize()
    return (out.cpu().numpy().reshape(case.B, case.Hq, 64),
            d["k"].cpu().numpy(), d["v"].cpu().numpy(), int(d["err"].item()))


@pytest.mark.parametrize("window", [0, 128])
def test_noalloc_matches_workspace_entry(gkv, cuda, window):
    import torch
    rng = np.random.default_rng(500 + window)
    for call, B in enumerate((48, 13)):
        L = rng.integers(0, 2500, size=B).astype(np.int32)
        L[0] = 0
        case = DecodeCase(B, 64, 8, L, window=window, scale=0.5, seed=501 + call + window)
        print(f"noalloc window={window} call={call} B={B}", flush=True)
        got = _run(case, gkv, torch, cuda, noalloc=True)
        ref = _run(case, gkv, torch, cuda, noalloc=False)
        assert got[3] == 0 and ref[3] == 0
        assert np.array_equal(got[1], ref[1]) and np.array_equal(got[2], ref[2])
        assert np.array_equal(from_pool(got[1].view(np.uint16), "k"), case.k_expect)
        assert np.array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
        bad, worst = allclose_report(got[0], case.oracle_out())
        assert bad == 0, f"{bad} outputs out of tolerance (max {worst:.3e})"
