"""libgkv.so on the CPU: it loads, exports every entry point of include/gkv.h,
its host RoPE table is the reference's, and it rejects bad arguments before
touching the GPU."""
import ctypes
import os
import re

import numpy as np

from oracle import kv_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "gkv.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gkv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_function(gkv):
    names = header_functions()
    assert len(names) >= 20
    lib = gkv.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(gkv.SIGNATURES), set(names) ^ set(gkv.SIGNATURES)


def test_status_strings(gkv):
    assert gkv.status_string(0) == "ok"
    for st in range(-6, 0):
        assert gkv.status_string(st) not in ("ok", "unknown status")
    assert gkv.lib().gkv_version().decode().count(".") == 2


def test_rope_table_bit_exact_vs_oracle_and_golden(gkv, golden):
    c, s = gkv.rope_table(4097)
    oc, os_ = O.rope_table(4097)
    assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    pos = golden["table_positions"]
    assert np.array_equal(c[pos].view(np.uint32), golden["table_cos"].view(np.uint32))
    assert np.array_equal(s[pos].view(np.uint32), golden["table_sin"].view(np.uint32))


def test_rope_table_without_scaling(gkv):
    c, s = gkv.rope_table(10, scaling_factor=1.0)
    inv = 1.0 / np.float32(150000.0) ** (np.arange(32, dtype=np.float32) * 2 / 64)
    assert np.allclose(c[9], np.cos(9 * inv), atol=1e-5)


def test_rope_table_rejects_bad_args(gkv):
    cfg = gkv.RopeConfig(**gkv.GPT_OSS_ROPE)
    buf = np.zeros(64, np.float32)
    assert gkv.lib().gkv_rope_table(ctypes.byref(cfg), -1, buf.ctypes.data, buf.ctypes.data) == gkv.GKV_ERR_ARG
    assert gkv.lib().gkv_rope_table(None, 1, buf.ctypes.data, buf.ctypes.data) == gkv.GKV_ERR_ARG
    cfg.head_dim = 63
    assert gkv.lib().gkv_rope_table(ctypes.byref(cfg), 1, buf.ctypes.data, buf.ctypes.data) == gkv.GKV_ERR_ARG


def _view(gkv, **kw):
    d = dict(k=1, v=1, block_table=1, table_stride=4, num_blocks=8, n_kv_heads=8, ring=0)
    d.update(kw)
    return gkv.CacheView(**d)


def test_append_argument_checks(gkv):
    L = gkv.lib()
    fake = 0x1000  # never dereferenced: the checks fail first
    args = lambda **o: dict(dict(stream=None, n=4, qkv=fake, stride=80 * 64, hq=64, cos=fake,
                                 sin=fake, pos=fake, seq=None, lens=None, view=_view(gkv),
                                 q_out=None, q_stride=0, kp=None, vp=None, err=None), **o)
    def call(a):
        return L.gkv_kv_append(a["stream"], a["n"], a["qkv"], a["stride"], a["hq"], a["cos"],
                               a["sin"], a["pos"], a["seq"], a["lens"], a["view"], a["q_out"],
                               a["q_stride"], a["kp"], a["vp"], a["err"])
    assert call(args(n=-1)) == gkv.GKV_ERR_ARG
    assert call(args(qkv=None)) == gkv.GKV_ERR_ARG
    assert call(args(stride=64)) == gkv.GKV_ERR_ARG            # row shorter than q|k|v
    assert call(args(hq=60)) == gkv.GKV_ERR_ARG                # not a multiple of Hkv
    assert call(args(view=_view(gkv, ring=100))) == gkv.GKV_ERR_UNSUPPORTED
    assert call(args(view=_view(gkv, num_blocks=0))) == gkv.GKV_ERR_ARG
    # a ring needs the lengths: rows W positions apart share a slot
    assert call(args(view=_view(gkv, ring=128))) == gkv.GKV_ERR_ARG
    assert call(args(n=0, view=_view(gkv, ring=128), lens=fake)) == gkv.GKV_OK
    assert call(args(n=0)) == gkv.GKV_OK                        # nothing to do


def test_qkv_append_argument_checks(gkv):
    L = gkv.lib()
    fake = 0x1000  # never dereferenced: the checks fail first
    N = 80 * 64
    args = lambda **o: dict(dict(n=4, x=fake, x_stride=2880, hidden=2880, w=fake, b=None, hq=64,
                                 cos=fake, sin=fake, pos=None, seq=None, lens=fake,
                                 view=_view(gkv), out=fake, out_stride=N, err=None), **o)
    def call(a):
        return L.gkv_qkv_append(None, a["n"], a["x"], a["x_stride"], a["hidden"], a["w"], a["b"],
                                a["hq"], a["cos"], a["sin"], a["pos"], a["seq"], a["lens"],
                                a["view"], a["out"], a["out_stride"], a["err"])
    assert call(args(n=-1)) == gkv.GKV_ERR_ARG
    assert call(args(x=None)) == gkv.GKV_ERR_ARG
    assert call(args(w=None)) == gkv.GKV_ERR_ARG
    assert call(args(hq=60)) == gkv.GKV_ERR_ARG                 # not a multiple of Hkv
    assert call(args(x_stride=2000)) == gkv.GKV_ERR_ARG         # row shorter than hidden
    assert call(args(out_stride=N - 1)) == gkv.GKV_ERR_ARG      # row shorter than q|k|v
    assert call(args(hidden=2900, x_stride=2904)) == gkv.GKV_ERR_UNSUPPORTED  # not 64k
    assert call(args(x_stride=2884)) == gkv.GKV_ERR_ARG         # 16-byte rows
    assert call(args(x=fake + 2)) == gkv.GKV_ERR_ARG            # 16-byte aligned
    assert call(args(cos=None)) == gkv.GKV_ERR_ARG              # the append needs the angles
    assert call(args(lens=None)) == gkv.GKV_ERR_ARG             # no way to find positions
    assert call(args(view=_view(gkv, ring=100))) == gkv.GKV_ERR_UNSUPPORTED
    assert call(args(view=_view(gkv, ring=128), pos=fake, lens=None)) == gkv.GKV_ERR_ARG
    assert call(args(view=_view(gkv, k=None, v=None), out=None)) == gkv.GKV_ERR_ARG  # no output
    assert call(args(n=0)) == gkv.GKV_OK                         # nothing to do
    # projection only: no cache, no angles needed
    assert call(args(n=0, view=_view(gkv, k=None, v=None), cos=None, sin=None)) == gkv.GKV_OK


def test_decode_argument_checks(gkv):
    L = gkv.lib()
    fake = 0x1000
    def call(B=4, hq=64, max_len=100, view=None, window=0, split=0, ws=None, ws_bytes=0,
             out_stride=4096, dtype=0, q=fake, lens=fake):
        return L.gkv_decode_attention(None, B, hq, q, 4096 + 1024, None, None, lens, max_len,
                                      view or _view(gkv), window, fake, split, ws, ws_bytes,
                                      fake, out_stride, dtype, None)
    assert call(B=-1) == gkv.GKV_ERR_ARG
    assert call(q=None) == gkv.GKV_ERR_ARG
    assert call(lens=None) == gkv.GKV_ERR_ARG
    assert call(hq=128 + 8) == gkv.GKV_ERR_UNSUPPORTED          # 17 query heads per kv head
    assert call(split=100) == gkv.GKV_ERR_ARG                   # not a multiple of 128
    assert call(B=8193) == gkv.GKV_ERR_UNSUPPORTED             # more sequences than one call takes
    assert call(out_stride=100) == gkv.GKV_ERR_ARG
    assert call(dtype=7) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, ring=128), window=0) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, ring=64), window=128) == gkv.GKV_ERR_ARG
    # a window is read from a ring of W slots, not from a full-length cache
    assert call(view=_view(gkv, ring=0), window=128) == gkv.GKV_ERR_UNSUPPORTED
    # a workspace of the advertised size is required
    need = gkv.workspace_bytes(4, 8, 5000)
    assert need > 0
    assert call(max_len=5000) == gkv.GKV_ERR_WORKSPACE
    assert call(max_len=5000, ws=fake, ws_bytes=need - 1) == gkv.GKV_ERR_WORKSPACE
    assert call(B=0, max_len=5000, ws=fake, ws_bytes=need) == gkv.GKV_OK
    # more fixed-size ranges than the workspace holds
    assert call(B=4, max_len=1 << 20, split=32, ws=fake, ws_bytes=need) == gkv.GKV_ERR_ARG


def test_planned_layer_argument_checks(gkv):
    """gkv_decode_layer_planned takes the modes 0-2 only; otherwise it checks
    as gkv_decode_layer does (B = 0: nothing to do)."""
    L = gkv.lib()
    fake = 0x1000  # never dereferenced: the checks fail first
    need = gkv.workspace_bytes(4, 8, 100)
    def call(plan, B=4, ws_bytes=need):
        return L.gkv_decode_layer_planned(None, B, 64, fake, 80 * 64, fake, fake, fake, 100,
                                          _view(gkv), 0, fake, 0, fake, ws_bytes, fake, 4096,
                                          0, None, plan)
    assert call(3) == gkv.GKV_ERR_ARG
    assert call(-1) == gkv.GKV_ERR_ARG
    for plan in (gkv.PLAN_NONE, gkv.PLAN_KEEP, gkv.PLAN_REUSE):
        assert call(plan, ws_bytes=need - 1) == gkv.GKV_ERR_WORKSPACE
        assert call(plan, B=0) == gkv.GKV_OK


def test_fp8_cache_needs_scales(gkv):
    """The prefill over a history and the appends need the e4m3 cache's
    scales."""
    L = gkv.lib()
    fake = 0x1000
    noscale = gkv.CacheView(fake, fake, fake, 8, 64, 8, 0, None, gkv.KV_FP8)
    st = L.gkv_prefill_paged(None, 1, fake, fake, 32, 64, fake, 5120, fake, fake, None, None,
                             noscale, fake, 0, fake, 4096, 0, None)
    assert st == gkv.GKV_ERR_ARG
    st = L.gkv_qkv_append(None, 4, fake, 2880, 2880, fake, None, 64, fake, fake, None, None,
                          fake, noscale, fake, 5120, None)
    assert st == gkv.GKV_ERR_ARG  # the e4m3 cache needs its scales
    bad = gkv.CacheView(fake, fake, fake, 8, 64, 8, 0, None, gkv.KV_FP8)  # scales required
    st = L.gkv_kv_append(None, 4, fake, 5120, 64, fake, fake, fake, None, fake, bad, None, 0,
                         None, None, None)
    assert st == gkv.GKV_ERR_ARG


def test_layer_combines_argument_checks(gkv):
    L = gkv.lib()
    assert L.gkv_decode_layer_combines(-1, 8, 100, 0, 0) == gkv.GKV_ERR_ARG
    assert L.gkv_decode_layer_combines(4, 0, 100, 0, 0) == gkv.GKV_ERR_ARG
    assert L.gkv_decode_layer_combines(4, 9, 100, 0, 0) == gkv.GKV_ERR_ARG
    assert L.gkv_decode_layer_combines(4, 8, 100, -1, 0) == gkv.GKV_ERR_ARG
    assert L.gkv_decode_layer_combines(4, 8, 100, 0, -32) == gkv.GKV_ERR_ARG
    assert L.gkv_decode_layer_combines(0, 8, 100, 128, 0) == 0  # nothing to launch


def test_workspace_formula(gkv):
    # plan (header + prefix sums + per range the sequence it starts inside of
    # and its start) and the combine's record per range; partial results of 2 segments per range for
    # up to 1024 ranges, 8 heads x (64 + 2) floats per kv head; then, for the
    # staged launches, block ids (1024 per range) and step records (512 per
    # range: ranges of up to 16384 tokens) and the query operands (2 KB per
    # sequence and kv head), then the kept plan (a 16-int key and 4 ints per
    # range); each part 256-byte aligned
    def a256(x):
        return (x + 255) // 256 * 256

    B, hkv = 512, 8
    parts = 2 * 1024 * hkv
    plan = a256((4 + B + 1 + 2 * 1024 + 1) * 4)  # + one range start per range, then T
    crec = a256(plan + 1024 * 16)                  # the combine's record per range
    fused = a256(crec + parts * (512 + 16) * 4)
    staged = (a256(1024 * 1024 * 4) + a256(1024 * 512 * 4) + a256(B * hkv * 2048)
              + a256((16 + 4 * 1024) * 4))
    assert gkv.workspace_bytes(B, hkv, 2049) == fused + staged
    # a window layer bounds the stream by the window
    assert gkv.workspace_bytes(B, hkv, 100000, window=128) == gkv.workspace_bytes(B, hkv, 128)


def test_engine_shim_header_compiles(tmp_path):
    """The C++ shim header parses as host C++ against gkv.h (no GPU needed)."""
    import shutil
    import subprocess
    cxx = shutil.which("g++")
    if cxx is None:
        import pytest
        pytest.skip("no g++")
    src = tmp_path / "shim.cpp"
    src.write_text('#include "gkv_engine.hpp"\nint main() { gkv_engine::PagedBatch b{}; '
                   'gkv_engine::PagedLayer l{}; (void)b; (void)l; return 0; }\n')
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([cxx, "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                        "-I", os.path.join(root, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_pool_calls_reject_null_and_bad_config(gkv):
    """Host-side argument checks of the pool (no device memory is touched)."""
    lib = gkv.lib()
    n = ctypes.c_int32()
    assert lib.gkv_pool_seq_alloc(None, ctypes.byref(n)) == gkv.GKV_ERR_ARG
    assert lib.gkv_pool_seq_reserve(None, 0, 10) == gkv.GKV_ERR_ARG
    assert lib.gkv_pool_seq_free(None, 0) == gkv.GKV_ERR_ARG
    assert lib.gkv_pool_sync(None, None) == gkv.GKV_ERR_ARG
    assert lib.gkv_pool_destroy(None) == gkv.GKV_ERR_ARG
    assert lib.gkv_pool_free_blocks(None) == -1
    assert lib.gkv_pool_num_blocks(None) == -1
    h = ctypes.c_void_p()
    for bad in (dict(n_layers=0), dict(head_dim=128), dict(window=20), dict(max_seqs=0)):
        cfg = dict(n_layers=2, n_kv_heads=8, head_dim=64, window=128, max_seqs=4,
                   max_seq_len=256, num_blocks=8, bytes_budget=0, shuffle_seed=0)
        cfg.update(bad)
        st = lib.gkv_pool_create(ctypes.byref(gkv.PoolConfig(*cfg.values())), ctypes.byref(h))
        assert st in (gkv.GKV_ERR_ARG, gkv.GKV_ERR_UNSUPPORTED), (bad, st)


def test_prefill_paged_argument_checks(gkv):
    L = gkv.lib()
    fake = 0x1000  # never dereferenced: the checks fail first
    def call(view=None, k=fake, v=fake, start=fake, window=0, B=2):
        return L.gkv_prefill_paged(None, B, fake, start, 100, 64, fake, 80 * 64, fake, fake, k, v,
                                   view if view is not None else _view(gkv, k=fake, v=fake), fake,
                                   window, fake,
                                   64 * 64, 0, None)
    assert call(B=-1) == gkv.GKV_ERR_ARG
    assert call(k=None, v=None, view=_view(gkv, k=None, v=None)) == gkv.GKV_ERR_ARG  # no keys
    assert call(v=None) == gkv.GKV_ERR_ARG                  # one of k, v
    assert call(view=_view(gkv, k=None, v=None)) == gkv.GKV_ERR_ARG  # a history needs the cache
    assert call(view=_view(gkv, k=fake, v=fake, ring=128), window=0) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, k=fake, v=fake, ring=128), window=64) == gkv.GKV_ERR_ARG
    # int8 V and e4m3 K/V need their scales (16-byte aligned), bf16 none; no other formats
    assert call(view=_view(gkv, k=fake, v=fake, v_format=1)) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, k=fake, v=fake, v_format=2)) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, k=fake, v=fake, v_format=1, v_scale=fake + 4)) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, k=fake, v=fake, v_format=0, v_scale=fake)) == gkv.GKV_ERR_ARG
    assert call(view=_view(gkv, k=fake, v=fake, v_format=3, v_scale=fake)) == gkv.GKV_ERR_ARG
    assert call(B=0) == gkv.GKV_OK
