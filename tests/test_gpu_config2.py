"""Config 2 at its full batch: B=512 sequences of context U[128, 2048],
H_q=64, H_kv=8, one full-attention layer of the gpt-oss-20b step through
gkv_decode_layer (append + split + combine), on a pool whose physical blocks
are handed out in shuffled order.

- The append over the whole batch, bit for bit: every byte of both pool
  arrays after the call (each new token at its slot, nothing else changed).
- The attention of 128 sampled sequences (the first, the last, the longest,
  the shortest, and random ones) against the CPU oracle within max-abs 2e-3 +
  rel 1e-2; every output of the batch finite, the device error word zero.
  At this batch the balanced ranges (one per resident workgroup) cut through
  several hundred sequences, whose pieces the combine launch merges; the
  sample holds such sequences (asserted from the plan's range size).
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


def test_config2_full_batch(gkv, cuda, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(20)
    B = 512
    L = rng.integers(128, 2048 + 1, size=B).astype(np.int32)
    print(f"config2 B={B} max_len={int(L.max()) + 1}", flush=True)
    P = PoolLayers(torch, gkv, L, n_layers=1, window=0, seed=21)
    try:
        ws = torch.empty(gkv.workspace_bytes(B, 8, P.max_len), dtype=torch.uint8, device=cuda)
        err = torch.zeros(1, dtype=torch.int32, device=cuda)
        sample = np.unique(np.concatenate([[0, B - 1, int(np.argmax(L)), int(np.argmin(L))],
                                           rng.choice(B, 124, replace=False)]))
        k0, v0 = P.snapshot(0)
        k_exp, v_exp = P.expected_after_append(0, k0, v0)
        del k0, v0
        out = torch.full((B, 64 * 64), float("nan"), dtype=torch.float32, device=cuda)
        view = P.views[0]
        gkv.decode_layer(P.t(P.qkv[0]), P.lens_d, P.max_len, view, P.t(P.sinks[0]), out,
                         P.cos_d, P.sin_d, window=0, workspace=ws, dev_err=err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        k1, v1 = P.snapshot(0)
        assert torch.equal(k1, k_exp), "K cache bytes differ"
        assert torch.equal(v1, v_exp), "V cache bytes differ"
        del k_exp, v_exp
        assert bool(torch.isfinite(out).all())
        # sequences of the sample that the ranges cut (their pieces merged by
        # the combine): stream offsets from the padded lengths, S from the plan
        plan = ws[:16].view(torch.int32).cpu().numpy()
        T, S, n_r = int(plan[0]), int(plan[1]), int(plan[2])
        n = (P.seq_lens + 31) // 32 * 32
        cu = np.concatenate([[0], np.cumsum(n)])
        assert T == cu[-1] and S == 0  # balanced ranges: range k starts at step k N / n_r
        starts = np.array([k * (T // 32) // n_r * 32 for k in range(n_r)])
        range_of = lambda p: int(np.searchsorted(starts, p, side="right")) - 1  # noqa: E731
        cut = [b for b in sample if range_of(cu[b]) != range_of(cu[b + 1] - 1)]
        print(f"{n_r} ranges of ~{T // n_r} tokens; {len(cut)} of {len(sample)} sampled "
              "sequences cut", flush=True)
        assert len(cut) >= 20
        got = out.cpu().numpy().reshape(B, 64, 64)[sample]
        ref = P.oracle_out(0, k1, v1, sample)
        bad, worst = allclose_report(got, ref)
        print(f"max abs err {worst:.2e} on {len(sample)} sequences", flush=True)
        assert bad == 0, f"{bad} outputs out of tolerance (max {worst:.3e})"
    finally:
        P.close()
