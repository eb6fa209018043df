"""GPU parity of the e4m3 K/V cache (GKV_KV_FP8) against the CPU oracle.

The append is bit-exact: every code byte of the K and V pools and every scale
equals orc_quantize_fp8 of the rotated key and of the value (NaN-poisoned
slots untouched). The attention reads the codes and scales and must match the
oracle's attention over the dequantized cache (scale * value(code)) within
max-abs 2e-3 + rel 1e-2, the contract tolerance.
"""
import numpy as np
import pytest

from kvcase import DecodeCase, allclose_report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def run(case, gkv, torch, device, layer_call):
    cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, device, cos, sin)
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring,
                          v_scale=dev["vs"], v_format=gkv.KV_FP8)
    max_len = int(case.seq_lens.max())
    ws = torch.empty(gkv.workspace_bytes(case.B, case.Hkv, max_len, case.window),
                     dtype=torch.uint8, device=device)
    out = torch.full((case.B, case.Hq * 64), float("nan"), dtype=torch.float32, device=device)
    if layer_call:
        gkv.decode_layer(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                         dev["cos"], dev["sin"], window=case.window, workspace=ws,
                         dev_err=dev["err"])
    else:
        gkv.kv_append(dev["qkv"], case.Hq, dev["cos"], dev["sin"], dev["pos"], view,
                      seq_lens=dev["seq_lens"], dev_err=dev["err"])
        gkv.decode_attention(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                             window=case.window, cos_tab=dev["cos"], sin_tab=dev["sin"],
                             workspace=ws, dev_err=dev["err"])
    torch.cuda.synchronize()
    return {"k": dev["k"].cpu().numpy(), "v": dev["v"].cpu().numpy(),
            "vs": dev["vs"].cpu().numpy(), "err": int(dev["err"].cpu().item()),
            "out": out.cpu().numpy().reshape(case.B, case.Hq, 64)}


def check(case, res):
    assert res["err"] == 0
    assert np.array_equal(res["k"], case.k_expect), "K codes differ"
    assert np.array_equal(res["v"], case.v_expect), "V codes differ"
    assert np.array_equal(res["vs"].view(np.uint32), case.vs_expect.view(np.uint32)), \
        "scales differ"
    assert np.isfinite(res["out"]).all()
    bad, worst = allclose_report(res["out"], case.oracle_out())
    assert bad == 0, f"{bad} outputs out of tolerance, max abs err {worst:.3e}"
    return worst


@pytest.mark.parametrize("layer_call", [False, True])
def test_fp8_full_layer(gkv, cuda, torch_mod, layer_call):
    rng = np.random.default_rng(80)
    B = 48
    L = rng.integers(128, 2048 + 1, size=B).astype(np.int32)
    L[:4] = [0, 1, 15, 31]
    case = DecodeCase(B, 64, 8, L, window=0, scale=0.5, seed=81, kv_fp8=True)
    worst = check(case, run(case, gkv, torch_mod, cuda, layer_call))
    print(f"fp8 full layer: max abs err {worst:.2e}")


@pytest.mark.parametrize("layer_call", [False, True])
def test_fp8_window_layer(gkv, cuda, torch_mod, layer_call):
    rng = np.random.default_rng(82)
    B = 300
    L = rng.integers(0, 4095 + 1, size=B).astype(np.int32)
    L[:4] = [0, 126, 127, 128]
    case = DecodeCase(B, 64, 8, L, window=128, scale=0.5, seed=83, kv_fp8=True)
    check(case, run(case, gkv, torch_mod, cuda, layer_call))


def test_fp8_large_scores_and_tiny_heads(gkv, cuda, torch_mod):
    """Large scores (scale 2.5, strong sinks) and heads of very different
    magnitudes: each token's scale stays its own."""
    rng = np.random.default_rng(84)
    L = rng.integers(1, 700, size=16).astype(np.int32)
    case = DecodeCase(16, 64, 8, L, window=0, scale=2.5, seed=85, sink_scale=6.0,
                      kv_fp8=True)
    check(case, run(case, gkv, torch_mod, cuda, False))


@pytest.mark.parametrize("hq,hkv,window", [(16, 2, 0), (12, 3, 128), (8, 4, 0), (8, 4, 128)])
def test_fp8_fewer_kv_heads(gkv, cuda, torch_mod, hq, hkv, window):
    """Fewer than 8 kv heads (the e4m3 launch's workgroup then has one wave per
    kv head) and group sizes 8, 4 and 2, on full and window layers."""
    rng = np.random.default_rng(86 + hkv)
    B = 40
    L = rng.integers(0, 1500, size=B).astype(np.int32)
    L[:3] = [0, 1, 127]
    case = DecodeCase(B, hq, hkv, L, window=window, scale=0.5, seed=87 + hkv, kv_fp8=True)
    check(case, run(case, gkv, torch_mod, cuda, True))
