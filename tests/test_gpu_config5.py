"""Config 5 at its full batch: B=1024 sequences of context U[1024, 3072],
H_q=64, H_kv=8, one 128-window (ring) layer and one full layer of the
gpt-oss-120b step, each through gkv_decode_layer (append + attention).

- The append is checked over the whole batch, bit for bit: every byte of both
  layers' pool arrays after the call (new tokens at their slots, nothing else
  changed).
- The attention of 96 sampled sequences (the first, the longest, the shortest
  and random ones) against the CPU oracle within max-abs 2e-3 + rel 1e-2;
  every output of the batch finite, the device error word zero.
- The split grid never exceeds the workgroups the GPU holds at once: with
  16384-token ranges, one range per resident slot covers the whole stream.
"""
import numpy as np
import pytest

from kvcase import allclose_report
from poolcase import PoolLayers

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def test_config5_full_batch_window_and_full_layer(gkv, cuda, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(5)
    B = 1024
    L = rng.integers(1024, 3072 + 1, size=B).astype(np.int32)
    L[1] = 3072  # the longest context of the config
    print(f"config5 B={B} max_len={int(L.max()) + 1}", flush=True)
    P = PoolLayers(torch, gkv, L, n_layers=2, window=128, seed=55)
    try:
        ws = torch.empty(gkv.workspace_bytes(B, 8, P.max_len), dtype=torch.uint8, device=cuda)
        err = torch.zeros(1, dtype=torch.int32, device=cuda)
        sample = np.unique(np.concatenate([[0, 1, int(np.argmin(L))],
                                           rng.choice(B, 93, replace=False)]))
        for li in range(2):
            k0, v0 = P.snapshot(li)
            k_exp, v_exp = P.expected_after_append(li, k0, v0)
            del k0, v0
            qkv = P.t(P.qkv[li])
            sinks = P.t(P.sinks[li])
            out = torch.full((B, 64 * 64), float("nan"), dtype=torch.float32, device=cuda)
            view = P.views[li]
            print(f"layer {li} window={view.ring}", flush=True)
            gkv.decode_layer(qkv, P.lens_d, P.max_len, view, sinks, out, P.cos_d, P.sin_d,
                             window=view.ring, workspace=ws, dev_err=err)
            torch.cuda.synchronize()
            assert int(err.item()) == 0
            k1, v1 = P.snapshot(li)
            assert torch.equal(k1, k_exp), f"layer {li}: K cache bytes differ"
            assert torch.equal(v1, v_exp), f"layer {li}: V cache bytes differ"
            del k_exp, v_exp
            assert bool(torch.isfinite(out).all())
            got = out.cpu().numpy().reshape(B, 64, 64)[sample]
            ref = P.oracle_out(li, k1, v1, sample)
            bad, worst = allclose_report(got, ref)
            print(f"layer {li}: max abs err {worst:.2e} on {len(sample)} sequences", flush=True)
            assert bad == 0, f"layer {li}: {bad} outputs out of tolerance (max {worst:.3e})"
            del k1, v1
    finally:
        P.close()
