"""The exact path on the CPU: its expf against the host C library on every
fp32 input, and the argument checks of its three entry points (which fail
before any GPU call)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CHECK = os.path.join(ROOT, "tests", "gkv_expf_check")


def test_expf_matches_host_libm_on_every_input():
    """gkv::expf_cpu_exact (csrc/exact_math.hpp), which the exact attention's
    softmax uses, equals the host's expf (the oracle's and run.cpp's, glibc)
    on all 2^32 fp32 bit patterns. A plausible slip (an unfused step, a table
    entry off by one ulp, a wrong coefficient) shows up as mismatches."""
    if not os.path.exists(CHECK):
        pytest.fail(f"{CHECK} is missing: run __graft_entry__.build() first")
    r = subprocess.run([CHECK, str(min(8, os.cpu_count() or 1))], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout, r.stdout


def test_exact_argument_checks(gkv):
    L = gkv.lib()
    fake = 0x1000  # never dereferenced: the checks fail first
    ARG, UNS = gkv.GKV_ERR_ARG, gkv.GKV_ERR_UNSUPPORTED

    def rope(**kw):
        a = dict(B=4, qkv=fake, row_stride=5120, cos=fake, sin=fake, pos=None, n_heads=72)
        a.update(kw)
        return L.gkv_rope_exact(None, a["B"], a["qkv"], a["row_stride"], a["cos"], a["sin"],
                                a["pos"], a["n_heads"])
    assert rope(B=0) == gkv.GKV_OK
    assert rope(B=-1) == ARG
    assert rope(qkv=None) == ARG
    assert rope(cos=None) == ARG
    assert rope(n_heads=0) == ARG
    assert rope(row_stride=72 * 64 - 1) == ARG

    def write(**kw):
        a = dict(B=4, qkv=fake, row_stride=5120, k_off=4096, v_off=4608, kc=fake, vc=fake,
                 slots=256, kv_dim=512, slot=3, pos=None, window=0)
        a.update(kw)
        return L.gkv_kv_write_exact(None, a["B"], a["qkv"], a["row_stride"], a["k_off"],
                                    a["v_off"], a["kc"], a["vc"], a["slots"], a["kv_dim"],
                                    a["slot"], a["pos"], a["window"], None)
    assert write(B=0) == gkv.GKV_OK
    assert write(kc=None) == ARG
    assert write(v_off=4609) == ARG           # V past the row
    assert write(slot=256) == ARG             # slot outside the cache
    assert write(slot=-1) == ARG
    assert write(window=128, slots=64) == ARG  # a ring smaller than the window
    assert write(slots=0) == ARG

    def attn(**kw):
        a = dict(B=4, hq=64, hkv=8, q=fake, q_stride=5120, kc=fake, vc=fake, slots=256,
                 sinks=fake, pos=10, positions=None, max_pos=0, window=0, out=fake,
                 out_stride=4096)
        a.update(kw)
        return L.gkv_attention_exact(None, a["B"], a["hq"], a["hkv"], a["q"], a["q_stride"],
                                     a["kc"], a["vc"], a["slots"], a["sinks"], a["pos"],
                                     a["positions"], a["max_pos"], a["window"], a["out"],
                                     a["out_stride"], None)
    assert attn(B=0) == gkv.GKV_OK
    assert attn(sinks=None) == ARG
    assert attn(hq=60) == ARG                 # not a multiple of the kv heads
    assert attn(hq=8 * 17, q_stride=8 * 17 * 64, out_stride=8 * 17 * 64) == UNS  # 17 per kv head
    assert attn(pos=256) == ARG               # a full layer's cache holds positions 0..255
    assert attn(pos=-1) == ARG
    assert attn(out_stride=4095) == ARG
    assert attn(window=128, slots=64) == ARG
