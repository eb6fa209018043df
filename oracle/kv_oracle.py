"""ctypes binding of the CPU oracle (liboracle.so) and of the reference build
(_ref/libref.so). TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
product path.

numpy in, numpy out. Every function mirrors the C function of the same name in
kv_oracle.h (which cites the reference lines it restates).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_long
_f = ctypes.c_float


class RopeCfg(ctypes.Structure):
    _fields_ = [("base", _f), ("head_dim", _i), ("scaling_factor", _f),
                ("initial_context_length", _f), ("ntk_beta", _f), ("ntk_alpha", _f)]


# gpt-oss (export_model_bin/gpt-oss-20b/config.json; run.cpp:582-583)
GPT_OSS_ROPE = dict(base=150000.0, head_dim=64, scaling_factor=32.0,
                    initial_context_length=4096.0, ntk_beta=32.0, ntk_alpha=1.0)


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.orc_yarn.argtypes = [ctypes.POINTER(RopeCfg), _vp, _vp]
        L.orc_cos_sin.argtypes = [ctypes.POINTER(RopeCfg), _i, _vp, _vp]
        L.orc_rope_table.argtypes = [ctypes.POINTER(RopeCfg), _i, _vp, _vp]
        L.orc_rotate.argtypes = [_vp, _vp, _vp, _i, _i]
        L.orc_f32_to_bf16_n.argtypes = [_vp, _vp, _l]
        L.orc_softmax.argtypes = [_vp, _i]
        L.orc_decode_attention.argtypes = [_i, _i, _i, _i, _vp, _l, _vp, _vp, _l, _vp, _vp, _i,
                                           _i, _vp, _l, _i]
        L.orc_decode_attention.restype = _i
        L.orc_prefill_attention.argtypes = [_i, _i, _i, _i, _vp, _vp, _l, _vp, _vp, _l, _vp, _i,
                                            _vp, _l, _i]
        L.orc_prefill_attention.restype = _i
        L.orc_quantize_v.argtypes = [_vp, _i, _i, _vp, _vp]
        L.orc_quantize_fp8.argtypes = [_vp, _i, _i, _vp, _vp]
        L.orc_fp8_value.argtypes = [ctypes.c_uint8]
        L.orc_fp8_value.restype = ctypes.c_float
        L.orc_linear.argtypes = [_i, _vp, _l, _vp, _vp, _i, _i, _vp, _l]
        L.orc_kv_append.argtypes = [_i, _i, _i, _i, _vp, _l, _vp, _vp, _vp, _vp, _vp, _vp, _vp]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own run.cpp functions (built by build_ref.sh)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH)
        R.ref_cos_sin.argtypes = [_i, _f, _i, _f, _f, _f, _f, _vp, _vp]
        R.ref_yarn.argtypes = [_f, _i, _f, _f, _f, _f, _vp, _vp]
        R.ref_rotate.argtypes = [_vp, _vp, _vp, _i, _i]
        R.ref_softmax.argtypes = [_vp, _i]
        R.ref_matmul_bias.argtypes = [_vp, _vp, _vp, _vp, _i, _i]
        R.ref_decode_one.argtypes = [_i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]
        R.ref_decode_one.restype = _i
        _ref = R
    return _ref


REF_Q8_PATH = os.path.join(os.path.dirname(REF_PATH), "libref_q8.so")
_ref_q8 = None


def ref_q8_available() -> bool:
    return os.path.exists(REF_Q8_PATH)


def ref_quantize_v(v: np.ndarray):
    """The reference's own quantize_v (attn_test.cpp:218-226) on one 64-value head."""
    global _ref_q8
    if _ref_q8 is None:
        _ref_q8 = ctypes.CDLL(REF_Q8_PATH)
        _ref_q8.ref_quantize_v.argtypes = [_vp, _vp, _vp]
    v = _f32(v)
    assert v.shape == (64,)
    codes = np.zeros(64, np.int8)
    scale = np.zeros(1, np.float32)
    _ref_q8.ref_quantize_v(_p(v), _p(codes), _p(scale))
    return codes, float(scale[0])


def _p(a: np.ndarray):
    return a.ctypes.data_as(_vp)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rope_cfg(**kw) -> RopeCfg:
    d = dict(GPT_OSS_ROPE)
    d.update(kw)
    return RopeCfg(**d)


def yarn(cfg: RopeCfg | None = None):
    cfg = cfg or rope_cfg()
    conc = np.zeros(1, np.float32)
    inv = np.zeros(cfg.head_dim // 2, np.float32)
    lib().orc_yarn(ctypes.byref(cfg), _p(conc), _p(inv))
    return float(conc[0]), inv


def rope_table(n_pos: int, cfg: RopeCfg | None = None):
    cfg = cfg or rope_cfg()
    half = cfg.head_dim // 2
    c = np.zeros((n_pos, half), np.float32)
    s = np.zeros((n_pos, half), np.float32)
    lib().orc_rope_table(ctypes.byref(cfg), n_pos, _p(c), _p(s))
    return c, s


def rotate(x: np.ndarray, cosv: np.ndarray, sinv: np.ndarray, head_dim: int = 64) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_rotate(_p(y), _p(_f32(cosv)), _p(_f32(sinv)), y.size // head_dim, head_dim)
    return y


def to_bf16(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_n(_p(x), _p(y), x.size)
    return y


def from_bf16(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def softmax(x: np.ndarray) -> np.ndarray:
    y = _f32(x).copy()
    lib().orc_softmax(_p(y), y.size)
    return y


def decode_attention(q, kc, vc, pos, sinks, window=0, ring=0, n_threads=0):
    """q [B, Hq, d] rotated; kc/vc [B, S, Hkv, d] (slot-indexed); pos [B]."""
    q = _f32(q)
    kc = _f32(kc)
    vc = _f32(vc)
    B, Hq, d = q.shape
    Hkv = kc.shape[2]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    sinks = _f32(sinks)
    out = np.zeros((B, Hq, d), np.float32)
    rc = lib().orc_decode_attention(B, Hq, Hkv, d, _p(q), Hq * d, _p(kc), _p(vc),
                                    kc.shape[1] * Hkv * d, _p(pos), _p(sinks), window, ring,
                                    _p(out), Hq * d, n_threads)
    if rc != 0:
        raise ValueError("orc_decode_attention: bad arguments")
    return out


def prefill_attention(cu_seqlens, q, k, v, sinks, window=0, n_threads=0):
    """q [T, Hq, d] rotated; k/v [T, Hkv, d]; cu_seqlens [B+1]."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    T, Hq, d = q.shape
    Hkv = k.shape[1]
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    out = np.zeros((T, Hq, d), np.float32)
    rc = lib().orc_prefill_attention(len(cu) - 1, Hq, Hkv, d, _p(cu), _p(q), Hq * d, _p(k),
                                     _p(v), Hkv * d, _p(_f32(sinks)), window, _p(out), Hq * d,
                                     n_threads)
    if rc != 0:
        raise ValueError("orc_prefill_attention: bad arguments")
    return out


def linear(x, w, bias=None):
    """x [rows, n_in], w [n_out, n_in] fp32 (bf16 values for the QKV
    projection), bias [n_out] or None -> [rows, n_out] fp32 (run.cpp matmul +
    bias add)."""
    x, w = _f32(x), _f32(w)
    rows, n_in = x.shape
    n_out = w.shape[0]
    assert w.shape[1] == n_in
    out = np.zeros((rows, n_out), np.float32)
    b = None if bias is None else _f32(bias)
    lib().orc_linear(rows, _p(x), n_in, _p(w), None if b is None else _p(b), n_in, n_out,
                     _p(out), n_out)
    return out


def kv_append(qkv, n_q_heads, n_kv_heads, cos_tab, sin_tab, pos, head_dim=64):
    """qkv [B, (Hq + 2 Hkv) d] fp32. Returns q_rot, k_rot, k_bf16, v_bf16."""
    qkv = _f32(qkv)
    B = qkv.shape[0]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    kv_dim = n_kv_heads * head_dim
    q_rot = np.zeros((B, n_q_heads, head_dim), np.float32)
    k_rot = np.zeros((B, n_kv_heads, head_dim), np.float32)
    kb = np.zeros((B, n_kv_heads, head_dim), np.uint16)
    vb = np.zeros((B, n_kv_heads, head_dim), np.uint16)
    lib().orc_kv_append(B, n_q_heads, n_kv_heads, head_dim, _p(qkv), qkv.shape[1],
                        _p(_f32(cos_tab)), _p(_f32(sin_tab)), _p(pos), _p(q_rot), _p(k_rot),
                        _p(kb), _p(vb))
    del kv_dim
    return q_rot, k_rot, kb, vb


def quantize_v(v, head_dim=64):
    """fp32 [..., n_heads, head_dim] -> (int8 codes, same shape; fp32 scales [..., n_heads])."""
    v = _f32(v)
    n_heads = v.size // head_dim
    codes = np.zeros(v.shape, np.int8)
    scales = np.zeros(v.shape[:-1], np.float32)
    lib().orc_quantize_v(_p(v), n_heads, head_dim, _p(codes), _p(scales))
    return codes, scales


def fp8_table() -> np.ndarray:
    """float32 [256]: the value of every e4m3 code (NaN for 0x7f, 0xff)."""
    return np.array([lib().orc_fp8_value(c) for c in range(256)], np.float32)


def quantize_fp8(x, head_dim=64):
    """fp32 [..., n_heads, head_dim] -> (uint8 e4m3 codes, same shape; fp32 scales
    [..., n_heads])."""
    x = _f32(x)
    n_heads = x.size // head_dim
    codes = np.zeros(x.shape, np.uint8)
    scales = np.zeros(x.shape[:-1], np.float32)
    lib().orc_quantize_fp8(_p(x), n_heads, head_dim, _p(codes), _p(scales))
    return codes, scales


def dequantize_fp8(codes, scales):
    """scale * value(code) in fp32, the values the e4m3 cache stands for."""
    return (fp8_table()[np.asarray(codes, np.uint8)] *
            np.asarray(scales, np.float32)[..., None]).astype(np.float32)


def dequantize_v(codes, scales):
    """scale * code in fp32, the values the int8 cache stands for."""
    return (np.asarray(codes, np.float32) * np.asarray(scales, np.float32)[..., None]).astype(
        np.float32)


# ---- the reference build -------------------------------------------------

def ref_cos_sin(pos: int, cfg: RopeCfg | None = None):
    cfg = cfg or rope_cfg()
    half = cfg.head_dim // 2
    c = np.zeros(half, np.float32)
    s = np.zeros(half, np.float32)
    ref().ref_cos_sin(pos, cfg.base, cfg.head_dim, cfg.scaling_factor,
                      cfg.initial_context_length, cfg.ntk_beta, cfg.ntk_alpha, _p(c), _p(s))
    return c, s


def ref_rotate(x, cosv, sinv, head_dim=64):
    y = _f32(x).copy()
    ref().ref_rotate(_p(y), _p(_f32(cosv).copy()), _p(_f32(sinv).copy()), y.size // head_dim,
                     head_dim)
    return y


def ref_softmax(x):
    y = _f32(x).copy()
    ref().ref_softmax(_p(y), y.size)
    return y


def ref_matmul_bias(x_row, w, bias=None):
    """run.cpp matmul of one input row plus the bias add (the reference's own code)."""
    x = _f32(x_row).copy()
    w = _f32(w).copy()
    n_out, n_in = w.shape
    out = np.zeros(n_out, np.float32)
    b = None if bias is None else _f32(bias).copy()
    ref().ref_matmul_bias(_p(out), _p(x), _p(w), None if b is None else _p(b), n_in, n_out)
    return out


def ref_decode_one(qkv_row, k_hist, v_hist, sinks, pos, n_q_heads, n_kv_heads, window=128,
                   window_layer=False, head_dim=64):
    """run.cpp forward() on one sequence. k_hist/v_hist [pos, Hkv*d], keys rotated."""
    out = np.zeros(n_q_heads * head_dim, np.float32)
    k_rot = np.zeros(n_kv_heads * head_dim, np.float32)
    kh = _f32(k_hist).reshape(-1)
    vh = _f32(v_hist).reshape(-1)
    if kh.size == 0:
        kh = np.zeros(1, np.float32)
        vh = np.zeros(1, np.float32)
    rc = ref().ref_decode_one(n_q_heads, n_kv_heads, head_dim, window, int(window_layer), pos,
                              _p(_f32(qkv_row)), _p(kh), _p(vh), _p(_f32(sinks)), _p(out),
                              _p(k_rot))
    if rc != 0:
        raise RuntimeError("ref_decode_one failed")
    return out.reshape(n_q_heads, head_dim), k_rot.reshape(n_kv_heads, head_dim)
