"""Seeded sweep of the decode path over shapes, formats and entry points.

Each case draws, from its seed: kv heads (1, 2, 4, 8) and query heads per kv
head (1 to 8), the batch (1 to 300), the context lengths (uniform, short,
long, or a mix with 0-token contexts), the window (none, 16, 32, 128, 256),
the cache format (bf16, int8 V, e4m3 K/V), the split (balanced or fixed
32-token multiples), the output type (fp32, bf16) and the entry point:
- "layer": gkv_decode_layer (append in the split's prologue);
- "two": gkv_kv_append, then gkv_decode_attention;
- "staged": gkv_kv_append, then gkv_decode_prepare / _split / _combine;
- "planned": gkv_decode_layer_planned keeping the plan, then a second call
  reusing it (the same inputs: the append rewrites the same bytes).
Every case checks the cache bytes bit for bit against the oracle's append
and the attention against the oracle within max-abs 2e-3 + rel 1e-2 (plus
bf16 rounding of the output for bf16 outputs), every output finite and the
device error word zero.
"""
import numpy as np
import pytest

from kvcase import DecodeCase, allclose_report

pytestmark = pytest.mark.gpu

N_CASES = 64


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def draw(seed):
    rng = np.random.default_rng(7000 + seed)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 3, 4, 5, 8]))
    fmt = str(rng.choice(["bf16", "int8", "fp8"]))
    window = int(rng.choice([0, 0, 16, 32, 128, 256]))
    B = int(rng.integers(1, 301))
    dist = str(rng.choice(["uniform", "short", "long", "mixed"]))
    if dist == "uniform":
        L = rng.integers(0, 2048, size=B)
    elif dist == "short":
        L = rng.integers(0, 64, size=B)
    elif dist == "long":
        L = rng.integers(1500, 3000, size=B)
    else:
        L = np.where(rng.random(B) < 0.2, 0, rng.integers(1, 2500, size=B))
    # at most ~300k cached (token, kv head) pairs, so a case builds in seconds
    ctx = np.minimum(L, window) if window else L
    keep = max(1, int(300_000 // (Hkv * max(1.0, float(ctx.mean())))))
    B = min(B, keep)
    L = L[:B]
    entry = str(rng.choice(["layer", "two", "staged", "planned"]))
    split = 0 if entry == "planned" and rng.random() < 0.5 else \
        int(rng.choice([0, 0, 0, 32, 64, 256, 1024]))
    # a fixed split may not need more than 1024 ranges (the workspace's bound)
    n_max = int(L.max()) + 1
    t_max = B * (-(-(min(n_max, window) if window else n_max) // 32) * 32)
    while split and -(-t_max // split) > 1024:
        split *= 2
    out_bf16 = bool(rng.random() < 0.3)
    scale = float(rng.choice([0.5, 0.5, 1.0, 2.0]))
    return dict(Hkv=Hkv, Hq=Hkv * G, fmt=fmt, window=window, B=B,
                L=np.asarray(L, np.int32), entry=entry, split=split, out_bf16=out_bf16,
                scale=scale, seed=8000 + seed)


def run_case(p, gkv, torch, device):
    case = DecodeCase(p["B"], p["Hq"], p["Hkv"], p["L"], window=p["window"], scale=p["scale"],
                      seed=p["seed"], v_int8=p["fmt"] == "int8", kv_fp8=p["fmt"] == "fp8")
    cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, device, cos, sin)
    v_format = {"bf16": gkv.V_BF16, "int8": gkv.V_INT8, "fp8": gkv.KV_FP8}[p["fmt"]]
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring,
                          v_scale=dev["vs"], v_format=v_format)
    max_len = int(case.seq_lens.max())
    ws = torch.empty(max(gkv.workspace_bytes(case.B, case.Hkv, max_len, case.window, p["split"]),
                         4), dtype=torch.uint8, device=device)
    dtype = torch.bfloat16 if p["out_bf16"] else torch.float32
    out = torch.full((case.B, case.Hq * 64), float("nan"), dtype=dtype, device=device)
    kw = dict(window=case.window, split_tokens=p["split"], workspace=ws, dev_err=dev["err"])
    entry = p["entry"]
    if entry == "layer":
        gkv.decode_layer(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                         dev["cos"], dev["sin"], **kw)
    elif entry == "planned":
        for plan in (gkv.PLAN_KEEP, gkv.PLAN_REUSE):
            out.fill_(float("nan"))
            gkv.decode_layer_planned(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"],
                                     out, dev["cos"], dev["sin"], plan, **kw)
    else:
        gkv.kv_append(dev["qkv"], case.Hq, dev["cos"], dev["sin"], dev["pos"], view,
                      seq_lens=dev["seq_lens"], dev_err=dev["err"])
        stages = ("both",) if entry == "two" else ("prepare", "split", "combine")
        for st in stages:
            gkv.decode_attention(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                                 cos_tab=dev["cos"], sin_tab=dev["sin"], stage=st, **kw)
    torch.cuda.synchronize()
    return case, {"k": dev["k"].cpu().numpy(), "v": dev["v"].cpu().numpy(),
                  "vs": None if dev["vs"] is None else dev["vs"].cpu().numpy(),
                  "err": int(dev["err"].cpu().item()),
                  "out": out.float().cpu().numpy().reshape(case.B, case.Hq, 64)}


@pytest.mark.parametrize("seed", range(N_CASES))
def test_decode_sweep(gkv, cuda, torch_mod, seed):
    from kvcase import to_pool
    p = draw(seed)
    print(f"sweep {seed}: B={p['B']} Hq={p['Hq']} Hkv={p['Hkv']} fmt={p['fmt']} "
          f"W={p['window']} entry={p['entry']} split={p['split']} bf16out={p['out_bf16']} "
          f"scale={p['scale']}", flush=True)
    case, res = run_case(p, gkv, torch_mod, cuda)
    assert res["err"] == 0, f"device error word {res['err']}"
    if p["fmt"] == "bf16":
        k_exp = to_pool(case.k_expect, "k").view(np.int16)
        v_exp = to_pool(case.v_expect, "v").view(np.int16)
        assert np.array_equal(res["k"].view(np.int16), k_exp), "K cache bytes differ"
        assert np.array_equal(res["v"].view(np.int16), v_exp), "V cache bytes differ"
    else:
        k_exp = case.k_expect if p["fmt"] == "fp8" else \
            to_pool(case.k_expect, "k").view(np.int16)
        assert np.array_equal(res["k"].view(k_exp.dtype), k_exp), "K cache bytes differ"
        assert np.array_equal(res["v"].view(case.v_expect.dtype), case.v_expect), \
            "V codes differ"
        assert np.array_equal(res["vs"].view(np.uint32), case.vs_expect.view(np.uint32)), \
            "scales differ"
    assert np.isfinite(res["out"]).all()
    ref = case.oracle_out()
    rtol = 1e-2 + (2.0 ** -8 if p["out_bf16"] else 0.0)
    bad, worst = allclose_report(res["out"], ref, 2e-3, rtol)
    print(f"  max abs err {worst:.2e}", flush=True)
    assert bad == 0, f"{bad} outputs out of tolerance, max abs err {worst:.3e}"
