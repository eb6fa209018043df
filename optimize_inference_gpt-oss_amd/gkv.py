"""ctypes binding of libgkv.so (include/gkv.h) for Python callers.

Device buffers are torch tensors (torch is used only for device memory and
streams); every call goes straight to the C ABI. A missing library raises:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# GKV_LIB overrides the library path (for trying a differently built libgkv.so).
LIB_PATH = os.environ.get("GKV_LIB") or os.path.join(HERE, "libgkv.so")

GKV_OK = 0
GKV_ERR_ARG = -1
GKV_ERR_UNSUPPORTED = -2
GKV_ERR_CAPACITY = -3
GKV_ERR_BLOCK = -4
GKV_ERR_HIP = -5
GKV_ERR_WORKSPACE = -6
DEVERR_BLOCK_ID = 1
DEVERR_LENGTH = 2
DEVERR_ALIGN = 4
DEVERR_RANGE = 8
F32 = 0
BF16 = 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_f = ctypes.c_float
_sz = ctypes.c_size_t


class CacheView(ctypes.Structure):
    _fields_ = [("k", _vp), ("v", _vp), ("block_table", _vp), ("table_stride", _i32),
                ("num_blocks", _i32), ("n_kv_heads", _i32), ("ring", _i32),
                ("v_scale", _vp), ("v_format", _i32)]


V_BF16, V_INT8, KV_FP8 = 0, 1, 2


def block_offsets(kind: str):
    """Element offsets inside one head's block of the pool (as the kernels in
    csrc/kv_append.hpp lay it out), as nested lists:
    - "k": [16 tokens][64 dims] of the bf16 K block (2 KB),
    - "v": [64 dims][16 tokens] of the bf16 V block (2 KB),
    - "v_int8": [64 dims][16 tokens] of the int8 V block (1 KB), also the e4m3 V block,
    - "k_fp8": [16 tokens][64 dims] of the e4m3 K block (1 KB)."""
    if kind == "k_fp8":
        return [[((d % 32) // 8 * 16 + t) * 16 + (d // 32) * 8 + d % 8 for d in range(64)]
                for t in range(16)]
    if kind == "k":
        return [[(d // 32) * 512 + ((d % 32) // 8 * 16 + t) * 8 + d % 8 for d in range(64)]
                for t in range(16)]
    if kind == "v":
        return [[(d // 32) * 512 + ((t // 4) * 16 + d % 16) * 8 + ((d // 16) % 2) * 4 + t % 4
                 for t in range(16)] for d in range(64)]
    if kind == "v_int8":
        return [[((d % 16) * 4 + t // 4) * 16 + (d // 16) * 4 + t % 4 for t in range(16)]
                for d in range(64)]
    raise ValueError(f"unknown block kind {kind!r}")


class RopeConfig(ctypes.Structure):
    _fields_ = [("base", _f), ("head_dim", _i32), ("scaling_factor", _f),
                ("initial_context_length", _f), ("ntk_beta", _f), ("ntk_alpha", _f)]


class PoolConfig(ctypes.Structure):
    _fields_ = [("n_layers", _i32), ("n_kv_heads", _i32), ("head_dim", _i32), ("window", _i32),
                ("max_seqs", _i32), ("max_seq_len", _i32), ("num_blocks", _i64),
                ("bytes_budget", _i64), ("shuffle_seed", _u64), ("v_format", _i32)]


GPT_OSS_ROPE = dict(base=150000.0, head_dim=64, scaling_factor=32.0,
                    initial_context_length=4096.0, ntk_beta=32.0, ntk_alpha=1.0)

# Every entry point of include/gkv.h: name -> (restype, argtypes)
SIGNATURES = {
    "gkv_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "gkv_version": (ctypes.c_char_p, []),
    "gkv_last_error": (ctypes.c_char_p, []),
    "gkv_rope_table": (ctypes.c_int, [ctypes.POINTER(RopeConfig), _i32, _vp, _vp]),
    "gkv_kv_append": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                                     CacheView, _vp, _i64, _vp, _vp, _vp]),
    "gkv_qkv_append": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i32, _vp, _vp, _i32, _vp, _vp,
                                      _vp, _vp, _vp, CacheView, _vp, _i64, _vp]),
    "gkv_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "gkv_decode_layer_combines": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32]),
    "gkv_decode_attention": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                            CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64,
                                            _i32, _vp]),
    "gkv_decode_prepare": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp]),
    "gkv_decode_layer": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp]),
    "gkv_decode_layer_planned": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp, _i32]),
    "gkv_decode_layer_split_planned": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp,
                                              _vp, _i32, CacheView, _i32, _vp, _i32, _vp, _sz,
                                              _vp, _i64, _i32, _vp, _i32]),
    "gkv_decode_layer_noalloc": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                               CacheView, _i32, _vp, _vp, _i64, _i32, _vp]),
    "gkv_decode_layer_split": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp]),
    "gkv_decode_layer_prepare": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp]),
    "gkv_decode_split": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp, _i32,
                                        CacheView, _i32, _vp, _i32, _vp, _sz, _vp, _i64, _i32,
                                        _vp]),
    "gkv_yardstick_decode_loads": (ctypes.c_int, [_vp, _i32, _i32, _vp, _i64, _vp, _vp, _vp,
                                                  _i32, CacheView, _i32, _vp, _i32, _vp, _sz,
                                                  _vp, _i64, _i32, _vp]),
    "gkv_yardstick_stream": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp]),
    "gkv_yardstick_gather": (ctypes.c_int, [_vp, _vp, _i64, _vp, _i32, _i32, _vp]),
    "gkv_decode_combine": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _i32,
                                          _vp, _sz, _vp, _i64, _i32]),
    "gkv_prefill_attention": (ctypes.c_int, [_vp, _i32, _vp, _i32, _i32, _i32, _vp, _i64, _vp,
                                             _vp, _vp, _vp, _vp, _i32, _vp, _i64, _i32]),
    "gkv_prefill_paged": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i32, _i32, _vp, _i64, _vp, _vp,
                                         _vp, _vp, CacheView, _vp, _i32, _vp, _i64, _i32, _vp]),
    "gkv_rope_exact": (ctypes.c_int, [_vp, _i32, _vp, _i64, _vp, _vp, _vp, _i32]),
    "gkv_kv_write_exact": (ctypes.c_int, [_vp, _i32, _vp, _i64, _i32, _i32, _vp, _vp, _i32, _i32,
                                          _i32, _vp, _i32, _vp]),
    "gkv_attention_exact": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _i64, _vp, _vp, _i32, _vp,
                                           _i32, _vp, _i32, _i32, _vp, _i64, _vp]),
    "gkv_pool_create": (ctypes.c_int, [ctypes.POINTER(PoolConfig), ctypes.POINTER(_vp)]),
    "gkv_pool_destroy": (ctypes.c_int, [_vp]),
    "gkv_pool_seq_alloc": (ctypes.c_int, [_vp, ctypes.POINTER(_i32)]),
    "gkv_pool_seq_reserve": (ctypes.c_int, [_vp, _i32, _i32]),
    "gkv_pool_seq_free": (ctypes.c_int, [_vp, _i32]),
    "gkv_pool_sync": (ctypes.c_int, [_vp, _vp]),
    "gkv_pool_layer_view": (ctypes.c_int, [_vp, _i32, ctypes.POINTER(CacheView)]),
    "gkv_pool_layer_view_from": (ctypes.c_int, [_vp, _i32, _i32, ctypes.POINTER(CacheView)]),
    "gkv_pool_free_blocks": (_i64, [_vp]),
    "gkv_pool_num_blocks": (_i64, [_vp]),
    "gkv_pool_device_bytes": (_i64, [_vp]),
    "gkv_pool_seq_blocks": (ctypes.c_int, [_vp, _i32, _vp, _i32, ctypes.POINTER(_i32)]),
}

_lib = None


class GkvError(RuntimeError):
    def __init__(self, fn: str, status: int):
        detail = lib().gkv_last_error().decode() if status == GKV_ERR_HIP else ""
        super().__init__(f"{fn}: {status_string(status)} ({status}) {detail}")
        self.status = status


def lib():
    """Load libgkv.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        # One HIP runtime per process: torch ships its own libamdhip64.so.7;
        # loading it first makes libgkv.so bind to that same runtime (its
        # NEEDED soname is already satisfied), so torch streams and device
        # pointers are valid in both.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build() first "
                               "(there is no fallback path)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().gkv_status_string(status).decode()


def check(fn: str, status: int) -> None:
    if status != GKV_OK:
        raise GkvError(fn, status)


def ptr(t) -> int | None:
    """Device (or host) address of a torch tensor / numpy array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


_hip = None


def hip_memcpy_d2d(dst: int, src: int, nbytes: int) -> None:
    """Device-to-device copy through the HIP runtime (plumbing for callers that
    fill or read pool arrays, which are not torch tensors)."""
    global _hip
    if _hip is None:
        lib()  # binds the process's HIP runtime first
        _hip = ctypes.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [_vp, _vp, _sz, ctypes.c_int]
    st = _hip.hipMemcpy(dst, src, nbytes, 3)  # hipMemcpyDeviceToDevice
    if st != 0:
        raise RuntimeError(f"hipMemcpy failed: {st}")


def stream_handle(stream=None) -> int | None:
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def rope_table(n_pos: int, **overrides):
    """Host numpy cos/sin tables [n_pos, head_dim/2] (gkv_rope_table)."""
    import numpy as np
    cfgd = dict(GPT_OSS_ROPE)
    cfgd.update(overrides)
    cfg = RopeConfig(**cfgd)
    half = cfg.head_dim // 2
    c = np.zeros((n_pos, half), np.float32)
    s = np.zeros((n_pos, half), np.float32)
    check("gkv_rope_table", lib().gkv_rope_table(ctypes.byref(cfg), n_pos, c.ctypes.data,
                                                 s.ctypes.data))
    return c, s


def cache_view(k, v, block_table, n_kv_heads: int, ring: int = 0, v_scale=None,
               v_format=None) -> CacheView:
    """View over torch tensors k [NB, Hkv, 16, 64], v [NB, Hkv, 64, 16] (bf16 or int16),
    block_table int32 [B, stride]. With v_scale (fp32 [NB, Hkv, 16]) the V cache is
    int8 codes [NB, Hkv, 1024] (GKV_V_INT8); v_format=KV_FP8: k and v are e4m3 codes
    [NB, Hkv, 1024] and v_scale fp32 [NB, Hkv, 32] (K scales, then V scales)."""
    if v_format is None:
        v_format = V_INT8 if v_scale is not None else V_BF16
    return CacheView(ptr(k), ptr(v), ptr(block_table), int(block_table.shape[1]),
                     int(k.shape[0]), int(n_kv_heads), int(ring), ptr(v_scale), int(v_format))


def kv_append(qkv, n_q_heads, cos_tab, sin_tab, row_pos, view: CacheView, row_seq=None,
              seq_lens=None, q_out=None, k_pack=None, v_pack=None, dev_err=None, stream=None):
    q_stride = q_out.stride(0) if q_out is not None else 0
    st = lib().gkv_kv_append(stream_handle(stream), qkv.shape[0], ptr(qkv), qkv.stride(0),
                             n_q_heads, ptr(cos_tab), ptr(sin_tab), ptr(row_pos), ptr(row_seq),
                             ptr(seq_lens), view, ptr(q_out), q_stride, ptr(k_pack), ptr(v_pack),
                             ptr(dev_err))
    check("gkv_kv_append", st)


def qkv_append(x, w_qkv, b_qkv, n_q_heads, cos_tab, sin_tab, view: CacheView | None,
               row_pos=None, row_seq=None, seq_lens=None, qkv_out=None, dev_err=None,
               stream=None, n_kv_heads=None):
    """gkv_qkv_append: qkv = x . w_qkv^T + b_qkv (x bf16 [rows, hidden], w_qkv bf16
    [(Hq + 2 Hkv) 64, hidden]) into qkv_out (fp32, optional), and the rotated K
    and the V of each row into the paged cache of `view` (optional)."""
    if view is None:  # projection only
        view = CacheView(n_kv_heads=n_kv_heads)
    out_stride = qkv_out.stride(0) if qkv_out is not None else 0
    st = lib().gkv_qkv_append(stream_handle(stream), x.shape[0], ptr(x), x.stride(0), x.shape[1],
                              ptr(w_qkv), ptr(b_qkv), n_q_heads, ptr(cos_tab), ptr(sin_tab),
                              ptr(row_pos), ptr(row_seq), ptr(seq_lens), view, ptr(qkv_out),
                              out_stride, ptr(dev_err))
    check("gkv_qkv_append", st)


def yardstick_stream(buf, n_workgroups, sink, stream=None):
    """gkv_yardstick_stream: read every byte of buf (a device tensor) once."""
    st = lib().gkv_yardstick_stream(stream_handle(stream), ptr(buf),
                                    buf.numel() * buf.element_size(), n_workgroups, ptr(sink))
    check("gkv_yardstick_stream", st)


def yardstick_gather(buf, block_ids, n_workgroups, sink, stream=None):
    """gkv_yardstick_gather: read the 2 KB blocks of buf listed in block_ids."""
    st = lib().gkv_yardstick_gather(stream_handle(stream), ptr(buf),
                                    buf.numel() * buf.element_size(), ptr(block_ids),
                                    block_ids.numel(), n_workgroups, ptr(sink))
    check("gkv_yardstick_gather", st)


def rope_exact(qkv, cos_tab, sin_tab, n_heads, positions=None, stream=None):
    """gkv_rope_exact: rotate heads 0..n_heads-1 of each fp32 row of qkv in place
    (run.cpp's rounding); row b at table row positions[b] (None: row 0)."""
    st = lib().gkv_rope_exact(stream_handle(stream), qkv.shape[0], ptr(qkv), qkv.stride(0),
                              ptr(cos_tab), ptr(sin_tab), ptr(positions), n_heads)
    check("gkv_rope_exact", st)


def kv_write_exact(qkv, k_off, v_off, kc, vc, kv_dim, slot=0, positions=None, window=0,
                   dev_err=None, stream=None):
    """gkv_kv_write_exact: each row's K and V into fp32 caches [B][slots][kv_dim]."""
    st = lib().gkv_kv_write_exact(stream_handle(stream), qkv.shape[0], ptr(qkv), qkv.stride(0),
                                  k_off, v_off, ptr(kc), ptr(vc), kc.shape[1], kv_dim, slot,
                                  ptr(positions), window, ptr(dev_err))
    check("gkv_kv_write_exact", st)


def attention_exact(q, n_q_heads, n_kv_heads, kc, vc, sinks, out, pos=0, positions=None,
                    max_pos=0, window=0, dev_err=None, stream=None):
    """gkv_attention_exact: decode attention over fp32 caches [B][slots][kv_dim],
    bit for bit with run.cpp's CPU forward."""
    st = lib().gkv_attention_exact(stream_handle(stream), q.shape[0], n_q_heads, n_kv_heads,
                                   ptr(q), q.stride(0), ptr(kc), ptr(vc), kc.shape[1],
                                   ptr(sinks), pos, ptr(positions), max_pos, window, ptr(out),
                                   out.stride(0), ptr(dev_err))
    check("gkv_attention_exact", st)


def workspace_bytes(B, n_kv_heads, max_seq_len, window=0, split_tokens=0) -> int:
    return lib().gkv_decode_workspace_bytes(B, n_kv_heads, max_seq_len, window, split_tokens)


def layer_combines(B, n_kv_heads, max_seq_len, window=0, split_tokens=0) -> bool:
    """gkv_decode_layer_combines: whether the layer launches the combine."""
    st = lib().gkv_decode_layer_combines(B, n_kv_heads, max_seq_len, window, split_tokens)
    if st < 0:
        check("gkv_decode_layer_combines", st)
    return st == 1


def decode_attention(q, seq_lens, max_seq_len, view: CacheView, sinks, out, window=0,
                     cos_tab=None, sin_tab=None, split_tokens=0, workspace=None, dev_err=None,
                     stream=None, stage="both"):
    import torch
    out_dtype = BF16 if out.dtype == torch.bfloat16 else F32
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    args_common = (stream_handle(stream), q.shape[0])
    if stage in ("both", "prepare", "split", "layer", "layer_prepare", "layer_split",
                 "yardstick_loads"):
        name = {"both": "gkv_decode_attention", "prepare": "gkv_decode_prepare",
                "split": "gkv_decode_split", "layer": "gkv_decode_layer",
                "layer_prepare": "gkv_decode_layer_prepare",
                "layer_split": "gkv_decode_layer_split",
                "yardstick_loads": "gkv_yardstick_decode_loads"}[stage]
        st = getattr(lib(), name)(*args_common, sinks.shape[0], ptr(q), q.stride(0),
                                  ptr(cos_tab), ptr(sin_tab), ptr(seq_lens), max_seq_len, view,
                                  window, ptr(sinks), split_tokens, ptr(workspace), ws_bytes,
                                  ptr(out), out.stride(0), out_dtype, ptr(dev_err))
        check(name, st)
    if stage == "combine":
        st = lib().gkv_decode_combine(*args_common, sinks.shape[0], view.n_kv_heads,
                                      ptr(seq_lens), max_seq_len, window, ptr(sinks),
                                      split_tokens, ptr(workspace), ws_bytes, ptr(out),
                                      out.stride(0), out_dtype)
        check("gkv_decode_combine", st)


def decode_layer(qkv, seq_lens, max_seq_len, view: CacheView, sinks, out, cos_tab, sin_tab,
                 window=0, split_tokens=0, workspace=None, dev_err=None, stream=None):
    """gkv_decode_layer: append of row b at position seq_lens[b]-1, then attention."""
    decode_attention(qkv, seq_lens, max_seq_len, view, sinks, out, window=window,
                     cos_tab=cos_tab, sin_tab=sin_tab, split_tokens=split_tokens,
                     workspace=workspace, dev_err=dev_err, stream=stream, stage="layer")


PLAN_NONE, PLAN_KEEP, PLAN_REUSE = 0, 1, 2
DEVERR_PLAN = 16


def decode_layer_planned(qkv, seq_lens, max_seq_len, view: CacheView, sinks, out, cos_tab,
                         sin_tab, plan, window=0, split_tokens=0, workspace=None, dev_err=None,
                         stream=None, split_only=False):
    """gkv_decode_layer_planned: gkv_decode_layer that keeps (PLAN_KEEP) or reuses
    (PLAN_REUSE) the split launch's plan in the workspace. split_only: the
    first launch alone (gkv_decode_layer_split_planned)."""
    import torch
    out_dtype = BF16 if out.dtype == torch.bfloat16 else F32
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    name = "gkv_decode_layer_split_planned" if split_only else "gkv_decode_layer_planned"
    st = getattr(lib(), name)(stream_handle(stream), qkv.shape[0], sinks.shape[0], ptr(qkv),
                              qkv.stride(0), ptr(cos_tab), ptr(sin_tab), ptr(seq_lens),
                              max_seq_len, view, window, ptr(sinks), split_tokens,
                              ptr(workspace), ws_bytes, ptr(out), out.stride(0), out_dtype,
                              ptr(dev_err), plan)
    check(name, st)


def decode_layer_noalloc(qkv, seq_lens, max_seq_len, view: CacheView, sinks, out, cos_tab,
                         sin_tab, window=0, dev_err=None, stream=None):
    """gkv_decode_layer_noalloc: gkv_decode_layer on the library's own scratch."""
    import torch
    out_dtype = BF16 if out.dtype == torch.bfloat16 else F32
    st = lib().gkv_decode_layer_noalloc(stream_handle(stream), qkv.shape[0], sinks.shape[0],
                                        ptr(qkv), qkv.stride(0), ptr(cos_tab), ptr(sin_tab),
                                        ptr(seq_lens), max_seq_len, view, window, ptr(sinks),
                                        ptr(out), out.stride(0), out_dtype, ptr(dev_err))
    check("gkv_decode_layer_noalloc", st)


def prefill_attention(cu_seqlens, max_len, q, k, v, sinks, out, n_kv_heads, window=0,
                      cos_tab=None, sin_tab=None, stream=None):
    """q: rotated rows, or (with cos_tab/sin_tab) the raw qkv rows, rotated on load."""
    import torch
    out_dtype = BF16 if out.dtype == torch.bfloat16 else F32
    st = lib().gkv_prefill_attention(stream_handle(stream), cu_seqlens.shape[0] - 1,
                                     ptr(cu_seqlens), max_len, sinks.shape[0], n_kv_heads,
                                     ptr(q), q.stride(0), ptr(cos_tab), ptr(sin_tab), ptr(k),
                                     ptr(v), ptr(sinks), window, ptr(out), out.stride(0),
                                     out_dtype)
    check("gkv_prefill_attention", st)


def prefill_paged(cu_seqlens, max_len, q, cache: CacheView, sinks, out, start_pos=None, k=None,
                  v=None, window=0, cos_tab=None, sin_tab=None, dev_err=None, stream=None):
    """gkv_prefill_paged: chunks continuing the sequences in `cache` (start_pos
    tokens each, multiples of 16); the chunk's keys from the packed rows k, v,
    or from the cache when they are None."""
    import torch
    out_dtype = BF16 if out.dtype == torch.bfloat16 else F32
    st = lib().gkv_prefill_paged(stream_handle(stream), cu_seqlens.shape[0] - 1, ptr(cu_seqlens),
                                 ptr(start_pos), max_len, sinks.shape[0], ptr(q), q.stride(0),
                                 ptr(cos_tab), ptr(sin_tab), ptr(k), ptr(v), cache, ptr(sinks),
                                 window, ptr(out), out.stride(0), out_dtype, ptr(dev_err))
    check("gkv_prefill_paged", st)


class Pool:
    """Paged KV pool (gkv_pool_*)."""

    def __init__(self, n_layers, n_kv_heads, max_seqs, max_seq_len, window=128, num_blocks=0,
                 bytes_budget=0, shuffle_seed=0, head_dim=64, v_format=0):
        self.cfg = PoolConfig(n_layers, n_kv_heads, head_dim, window, max_seqs, max_seq_len,
                              num_blocks, bytes_budget, shuffle_seed, v_format)
        h = _vp()
        check("gkv_pool_create", lib().gkv_pool_create(ctypes.byref(self.cfg), ctypes.byref(h)))
        self.h = h

    def close(self):
        if self.h:
            lib().gkv_pool_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def seq_alloc(self) -> int:
        s = _i32()
        check("gkv_pool_seq_alloc", lib().gkv_pool_seq_alloc(self.h, ctypes.byref(s)))
        return s.value

    def reserve(self, seq: int, seq_len: int) -> int:
        return lib().gkv_pool_seq_reserve(self.h, seq, seq_len)

    def free(self, seq: int) -> int:
        return lib().gkv_pool_seq_free(self.h, seq)

    def sync(self, stream=None):
        check("gkv_pool_sync", lib().gkv_pool_sync(self.h, stream_handle(stream)))

    def view(self, layer: int, first_seq: int = 0) -> CacheView:
        v = CacheView()
        check("gkv_pool_layer_view_from",
              lib().gkv_pool_layer_view_from(self.h, layer, first_seq, ctypes.byref(v)))
        return v

    def free_blocks(self) -> int:
        return lib().gkv_pool_free_blocks(self.h)

    def num_blocks(self) -> int:
        return lib().gkv_pool_num_blocks(self.h)

    def device_bytes(self) -> int:
        return lib().gkv_pool_device_bytes(self.h)

    def seq_blocks(self, seq: int):
        import numpy as np
        n = _i32()
        check("gkv_pool_seq_blocks",
              lib().gkv_pool_seq_blocks(self.h, seq, None, 0, ctypes.byref(n)))
        out = np.zeros(max(n.value, 1), np.int32)
        check("gkv_pool_seq_blocks",
              lib().gkv_pool_seq_blocks(self.h, seq, out.ctypes.data, n.value, ctypes.byref(n)))
        return out[:n.value]
