"""The C++ engine shim (include/gkv_engine.hpp) driven the way the reference
engine drives its attention: a C++ decode loop (tests/engine_demo.cpp, built by
build()) calls rope_kv_bf16 + attention_bf16_chunk64 (or, on the int8-V cache,
the engine's own pair rope_kv_bf16 + attention_q8v_chunk64) per layer and step over
the paged pool (one window layer with a wrapping 32-slot ring, one full
layer). Every step's bf16 output is compared with the CPU oracle, which keeps
the history by position: max-abs 2e-3 + rel 1e-2, plus bf16 output rounding.
The "project" form also runs the QKV projection through gemm_bf16_rope_kv.
"""
import os
import subprocess

import numpy as np
import pytest

from kvcase import allclose_report

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(ROOT, "tests", "gkv_engine_demo")


def _bf16_values(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


@pytest.mark.parametrize("mode,v_int8", [(None, False), ("fused", False), ("fused", True),
                                         ("planned", False), ("project", False),
                                         ("q8v", True)])
def test_engine_shim_decode_loop(oracle, cuda, tmp_path, mode, v_int8):
    """mode None: rope_kv_bf16 + attention_bf16_chunk64; "q8v": rope_kv_bf16 +
    attention_q8v_chunk64 in the reference's argument order; "fused": the one-call
    rope_kv_attention_bf16; "planned": the same over four layers, the first of
    each kind keeping its plan and the others reusing it; "project": the qkv
    rows come from the layer input
    through gemm_bf16_rope_kv (projection with the append in its epilogue),
    and the oracle's rows from orc_linear (run.cpp matmul + bias)."""
    if not os.path.exists(DEMO):
        pytest.fail("gkv_engine_demo is not built (run __graft_entry__.build())")
    P, B, Hq, Hkv, NL, W = 40, 3, 64, 8, 4 if mode == "planned" else 2, 32
    rng = np.random.default_rng(2024)
    QKV = (Hq + 2 * Hkv) * 64
    qkv = (rng.standard_normal((P, NL, B, QKV)) * 0.5).astype(np.float32)
    sinks = rng.standard_normal((NL, Hq)).astype(np.float32)
    H = 192
    if mode == "project":
        x = _bf16_values(rng.standard_normal((P, NL, B, H)))
        w = _bf16_values(rng.standard_normal((NL, QKV, H)) * 0.04)
        bias = (rng.standard_normal((NL, QKV)) * 0.1).astype(np.float32)
        for p in range(P):
            for l in range(NL):
                qkv[p, l] = oracle.linear(x[p, l], w[l], bias[l])
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        np.array([P, B, Hq, Hkv, NL, W, 1 if v_int8 else 0], np.int32).tofile(f)
        qkv.tofile(f)
        sinks.tofile(f)
        if mode == "project":
            np.array([H], np.int32).tofile(f)
            for a in (x, w):
                (a.view(np.uint32) >> 16).astype(np.uint16).tofile(f)
            bias.tofile(f)
    cmd = [DEMO, str(inp), str(outp)] + ([mode] if mode else [])
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=90)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(outp, np.uint16).reshape(P, NL, B, Hq, 64)
    got = oracle.from_bf16(got)

    cos, sin = oracle.rope_table(P)
    for l in range(NL):
        window = W if l % 2 == 0 else 0
        kc = np.zeros((B, P, Hkv, 64), np.float32)
        vc = np.zeros((B, P, Hkv, 64), np.float32)
        for p in range(P):
            pos = np.full(B, p, np.int32)
            q_rot, _, kb, vb = oracle.kv_append(qkv[p, l], Hq, Hkv, cos, sin, pos)
            kc[:, p] = oracle.from_bf16(kb)
            if v_int8:
                v_new = qkv[p, l][:, (Hq + Hkv) * 64:].reshape(B, Hkv, 64)
                vc[:, p] = oracle.dequantize_v(*oracle.quantize_v(v_new))
            else:
                vc[:, p] = oracle.from_bf16(vb)
            ref = oracle.decode_attention(q_rot, kc[:, :p + 1], vc[:, :p + 1], pos, sinks[l],
                                          window=window)
            n_bad, max_err = allclose_report(got[p, l], ref, 2e-3, 1e-2 + 2 ** -8)
            assert n_bad == 0, f"layer {l} step {p}: {n_bad} bad, max err {max_err}"


@pytest.mark.parametrize("mode,v_int8", [(None, True), ("q8v", False)])
def test_engine_shim_rejects_mismatched_cache(cuda, tmp_path, mode, v_int8):
    """attention_bf16_chunk64 on an int8-V pool, and attention_q8v_chunk64 on a
    bf16 one, fail loudly (the shim prints and exits, as the reference's
    HIP_CHECK does) instead of reading the cache in the wrong format."""
    if not os.path.exists(DEMO):
        pytest.fail("gkv_engine_demo is not built (run __graft_entry__.build())")
    P, B, Hq, Hkv, NL, W = 2, 1, 64, 8, 2, 32
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        np.array([P, B, Hq, Hkv, NL, W, 1 if v_int8 else 0], np.int32).tofile(f)
        np.zeros((P, NL, B, (Hq + 2 * Hkv) * 64), np.float32).tofile(f)
        np.zeros((NL, Hq), np.float32).tofile(f)
    cmd = [DEMO, str(inp), str(outp)] + ([mode] if mode else [])
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=90)
    assert r.returncode != 0
    assert "attention_" in r.stderr and "bad argument" in r.stderr, r.stderr


def test_engine_shim_exact_loop(oracle, cuda, tmp_path):
    """The GPTOSS_EXACT trio through the shim (rope_exact, kv_write_kernel,
    attention_exact in layer_attention's order, fp32 caches per layer, a
    32-slot ring on the window layer): every step's fp32 output equals the
    CPU oracle's bit for bit."""
    if not os.path.exists(DEMO):
        pytest.fail("gkv_engine_demo is not built (run __graft_entry__.build())")
    P, B, Hq, Hkv, NL, W = 40, 3, 64, 8, 2, 32
    rng = np.random.default_rng(2025)
    QKV = (Hq + 2 * Hkv) * 64
    qkv = (rng.standard_normal((P, NL, B, QKV)) * 0.5).astype(np.float32)
    sinks = rng.standard_normal((NL, Hq)).astype(np.float32)
    inp, outp = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        np.array([P, B, Hq, Hkv, NL, W, 0], np.int32).tofile(f)
        qkv.tofile(f)
        sinks.tofile(f)
    r = subprocess.run([DEMO, str(inp), str(outp), "exact"], capture_output=True, text=True,
                       timeout=90)
    assert r.returncode == 0, r.stderr
    got = np.fromfile(outp, np.float32).reshape(P, NL, B, Hq, 64)
    cos, sin = oracle.rope_table(P)
    for l in range(NL):
        window = W if l % 2 == 0 else 0
        kc = np.zeros((B, P, Hkv, 64), np.float32)
        vc = np.zeros((B, P, Hkv, 64), np.float32)
        for p in range(P):
            pos = np.full(B, p, np.int32)
            q_rot, k_rot, _, _ = oracle.kv_append(qkv[p, l], Hq, Hkv, cos, sin, pos)
            kc[:, p] = k_rot
            vc[:, p] = qkv[p, l][:, (Hq + Hkv) * 64:].reshape(B, Hkv, 64)
            ref = oracle.decode_attention(q_rot, kc[:, :p + 1], vc[:, :p + 1], pos, sinks[l],
                                          window=window)
            g = np.ascontiguousarray(got[p, l]).view(np.uint32)
            w = np.ascontiguousarray(ref).view(np.uint32)
            assert (g == w).all(), f"layer {l} step {p}: {(g != w).sum()} values differ"
