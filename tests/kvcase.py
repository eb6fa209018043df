"""Seeded decode cases: a paged cache with history, the new token's qkv row,
and what the CPU oracle says the append and the attention must produce.

The physical placement is a random permutation of block ids; every slot and
block that holds no token is poisoned with bf16 NaN (0x7fc0), so a kernel that
reads or writes outside its tokens shows up as a NaN or a changed byte.
"""
from __future__ import annotations

import numpy as np

from oracle import kv_oracle as O

D = 64
BT = 16
BF16_NAN = 0x7FC0
INT8_POISON = 0x55  # codes of int8-V slots that hold no token


def v_int8_offsets(t):
    """Byte offsets of dims 0..63 of token t (0..15) in a head's 1 KB int8 V block
    (t an int, or an array [..., 1] for one row of offsets per token)."""
    d = np.arange(D)
    return ((d % 16) * 4 + t // 4) * 16 + (d // 16) * 4 + t % 4


def k_block_offsets():
    """[16, 64]: element offset of (token t, dim d) in a head's bf16 K block.
    Lane kg*16 + t of the attention kernel loads 8 elements at lane*8 (+512 for
    dims 32..63): dims 32m + 8kg .. +7 of token t."""
    t = np.arange(BT)[:, None]
    d = np.arange(D)[None, :]
    return (d // 32) * 512 + ((d % 32) // 8 * 16 + t) * 8 + d % 8


def v_block_offsets():
    """[64, 16]: element offset of (dim d, token t) in a head's bf16 V block.
    Lane kg*16 + i loads 8 elements at lane*8 (+512 for half h): tokens
    4kg .. 4kg+3 of dim i + 32h, then of dim i + 32h + 16."""
    d = np.arange(D)[:, None]
    t = np.arange(BT)[None, :]
    return (d // 32) * 512 + ((t // 4) * 16 + d % 16) * 8 + ((d // 16) % 2) * 4 + t % 4


def k_fp8_offsets(t):
    """Byte offsets of dims 0..63 of token t in a head's 1 KB e4m3 K block: lane
    kg*16 + t loads 16 bytes at lane*16, dims 8kg..8kg+7 then 32+8kg..+7 (t an
    int, or an array [..., 1])."""
    d = np.arange(D)
    return ((d % 32) // 8 * 16 + t) * 16 + (d // 32) * 8 + d % 8


FP8_NAN = 0x7F  # e4m3 NaN: the poison of slots that hold no token


_K_OFF = k_block_offsets().reshape(-1)
_V_OFF = v_block_offsets().reshape(-1)


def to_pool(x, kind):
    """Logical blocks ([..., 16, 64] K or [..., 64, 16] V) -> pool bytes [..., 1024]."""
    off = _K_OFF if kind == "k" else _V_OFF
    out = np.empty(x.shape[:-2] + (BT * D,), x.dtype)
    out[..., off] = x.reshape(x.shape[:-2] + (BT * D,))
    return out


def from_pool(p, kind):
    """Pool bytes [..., 1024] (or any [..., 16, 64]-sized trailing dims) -> logical blocks."""
    p = p.reshape(p.shape[:-2] + (BT * D,)) if p.shape[-1] != BT * D else p
    off = _K_OFF if kind == "k" else _V_OFF
    shape = (BT, D) if kind == "k" else (D, BT)
    return p[..., off].reshape(p.shape[:-1] + shape)


class DecodeCase:
    def __init__(self, B, n_q_heads, n_kv_heads, ctx_lens, window=0, scale=1.0, seed=0,
                 extra_blocks=7, rope_rows=None, sink_scale=1.0, v_int8=False, kv_fp8=False):
        rng = np.random.default_rng(seed)
        self.v_int8 = v_int8
        self.kv_fp8 = kv_fp8
        self.B, self.Hq, self.Hkv = B, n_q_heads, n_kv_heads
        self.window = window
        self.ring = window
        self.L = np.asarray(ctx_lens, np.int32)      # context before the append
        assert self.L.shape == (B,)
        self.pos = self.L.copy()                     # position of the new token
        self.seq_lens = self.L + 1
        kvd = n_kv_heads * D
        self.row_width = (n_q_heads + 2 * n_kv_heads) * D
        self.qkv = (rng.standard_normal((B, self.row_width)) * scale).astype(np.float32)
        self.sinks = (rng.standard_normal(n_q_heads) * sink_scale).astype(np.float32)
        n_rope = rope_rows if rope_rows is not None else int(self.pos.max()) + 1
        self.cos, self.sin = O.rope_table(n_rope)

        # Block tables.
        if self.ring:
            per_seq = np.full(B, self.ring // BT, np.int32)
        else:
            per_seq = (self.seq_lens + BT - 1) // BT
        self.table_stride = int(per_seq.max())
        self.num_blocks = int(per_seq.sum()) + extra_blocks
        ids = rng.permutation(self.num_blocks).astype(np.int32)
        self.table = np.full((B, self.table_stride), -1, np.int32)
        o = 0
        for b in range(B):
            self.table[b, :per_seq[b]] = ids[o:o + per_seq[b]]
            o += per_seq[b]

        # Caches, poisoned.
        self.k = np.full((self.num_blocks, n_kv_heads, BT, D), BF16_NAN, np.uint16)
        if kv_fp8:
            self.k = np.full((self.num_blocks, n_kv_heads, BT * D), FP8_NAN, np.uint8)
            self.v = np.full((self.num_blocks, n_kv_heads, BT * D), FP8_NAN, np.uint8)
            self.vs = np.full((self.num_blocks, n_kv_heads, 2 * BT), np.nan, np.float32)
        elif v_int8:
            self.v = np.full((self.num_blocks, n_kv_heads, BT * D), INT8_POISON, np.int8)
            self.vs = np.full((self.num_blocks, n_kv_heads, BT), np.nan, np.float32)
        else:
            self.v = np.full((self.num_blocks, n_kv_heads, D, BT), BF16_NAN, np.uint16)
            self.vs = None
        # Oracle's logical cache (slot-indexed fp32 of the bf16 values).
        S = self.ring if self.ring else int(self.seq_lens.max())
        self.S = S
        self.kc = np.zeros((B, S, n_kv_heads, D), np.float32)
        self.vc = np.zeros((B, S, n_kv_heads, D), np.float32)
        for b in range(B):
            L = int(self.L[b])
            if self.ring:
                # Tokens the ring holds before this append: L-W .. L-1 (the
                # oldest is overwritten by the new token).
                t_hist = np.arange(max(0, L - self.ring), L)
            else:
                t_hist = np.arange(0, L)
            if len(t_hist) == 0:
                continue
            kh = O.to_bf16(rng.standard_normal((len(t_hist), n_kv_heads, D)) * scale)
            vf = (rng.standard_normal((len(t_hist), n_kv_heads, D)) * scale).astype(np.float32)
            slots = t_hist % self.ring if self.ring else t_hist
            if kv_fp8:
                kf = (rng.standard_normal((len(t_hist), n_kv_heads, D)) * scale).astype(np.float32)
                kcodes, kscales = O.quantize_fp8(kf)
                vcodes, vscales = O.quantize_fp8(vf)
                self._place_f8(self.k, self.v, self.vs, b, slots, kcodes, kscales, vcodes,
                               vscales)
                self.kc[b, slots] = O.dequantize_fp8(kcodes, kscales)
                self.vc[b, slots] = O.dequantize_fp8(vcodes, vscales)
                continue
            if v_int8:
                codes, scales = O.quantize_v(vf)
                self._place_k(self.k, b, slots, kh)
                self._place_v8(self.v, self.vs, b, slots, codes, scales)
                self.vc[b, slots] = O.dequantize_v(codes, scales)
            else:
                vh = O.to_bf16(vf)
                self._place(b, slots, kh, vh)
                self.vc[b, slots] = O.from_bf16(vh)
            self.kc[b, slots] = O.from_bf16(kh)

        # The append, per the oracle.
        q_rot, k_rot, kb, vb = O.kv_append(self.qkv, n_q_heads, n_kv_heads, self.cos, self.sin,
                                           self.pos)
        self.q_rot = q_rot
        self.k_expect = self.k.copy()
        self.v_expect = self.v.copy()
        self.vs_expect = self.vs.copy() if (v_int8 or kv_fp8) else None
        v_new = self.qkv[:, (n_q_heads + n_kv_heads) * D:].reshape(B, n_kv_heads, D)
        k_new = np.asarray(k_rot, np.float32).reshape(B, n_kv_heads, D)
        for b in range(B):
            slot = int(self.pos[b] % self.ring) if self.ring else int(self.pos[b])
            phys = self.table[b, slot // BT]
            if kv_fp8:
                kcodes, kscales = O.quantize_fp8(k_new[b])
                vcodes, vscales = O.quantize_fp8(v_new[b])
                self._place_f8(self.k_expect, self.v_expect, self.vs_expect, b,
                               np.array([slot]), kcodes[None], kscales[None], vcodes[None],
                               vscales[None])
                self.kc[b, slot] = O.dequantize_fp8(kcodes, kscales)
                self.vc[b, slot] = O.dequantize_fp8(vcodes, vscales)
                continue
            self.k_expect[phys, :, slot % BT, :] = kb[b]
            self.kc[b, slot] = O.from_bf16(kb[b])
            if v_int8:
                codes, scales = O.quantize_v(v_new[b])
                self._place_v8(self.v_expect, self.vs_expect, b, np.array([slot]), codes[None],
                               scales[None])
                self.vc[b, slot] = O.dequantize_v(codes, scales)
            else:
                self.v_expect[phys, :, :, slot % BT] = vb[b]
                self.vc[b, slot] = O.from_bf16(vb[b])
        del kvd

    def _place_k(self, k, b, slots, kh):
        phys = self.table[b, slots // BT]
        k[phys, :, slots % BT, :] = kh

    def _slots(self, b, slots):
        """Physical block [n, 1, 1], token in block [n] and head index [1, Hkv, 1]
        of the listed slots of sequence b."""
        slots = np.asarray(slots)
        phys = self.table[b, slots // BT].astype(np.int64)[:, None, None]
        return phys, slots % BT, np.arange(self.Hkv)[None, :, None]

    def _place_v8(self, v, vs, b, slots, codes, scales):
        """codes [n, Hkv, 64] int8, scales [n, Hkv] -> the int8 block layout."""
        phys, t, g = self._slots(b, slots)
        v[phys, g, v_int8_offsets(t[:, None])[:, None, :]] = codes
        vs[phys[:, 0, 0], :, t] = scales

    def _place_f8(self, k, v, s, b, slots, kcodes, kscales, vcodes, vscales):
        """e4m3 codes [n, Hkv, 64] and scales [n, Hkv] -> the e4m3 block layouts,
        K scales at token t, V scales at 16 + t."""
        phys, t, g = self._slots(b, slots)
        k[phys, g, k_fp8_offsets(t[:, None])[:, None, :]] = kcodes
        v[phys, g, v_int8_offsets(t[:, None])[:, None, :]] = vcodes
        s[phys[:, 0, 0], :, t] = kscales
        s[phys[:, 0, 0], :, BT + t] = vscales

    def _place(self, b, slots, kh, vh):
        phys = self.table[b, slots // BT]
        off = slots % BT
        self.k[phys, :, off, :] = kh
        # v[phys, g, :, off] = vh[j, g, :]
        self.v[phys, :, :, off] = vh

    def oracle_out(self, n_threads=0):
        return O.decode_attention(self.q_rot, self.kc, self.vc, self.pos, self.sinks,
                                  window=self.window, ring=self.ring, n_threads=n_threads)

    # ---- device side ------------------------------------------------------
    def to_device(self, torch, device, cos=None, sin=None):
        """Tensors for the GPU path. cos/sin: the product's host table (defaults
        to the oracle's, which is bit-identical)."""
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        dev = {
            "qkv": t(self.qkv),
            "sinks": t(self.sinks),
            "cos": t(self.cos if cos is None else cos),
            "sin": t(self.sin if sin is None else sin),
            "pos": t(self.pos),
            "seq_lens": t(self.seq_lens),
            "table": t(self.table),
            "k": t(self.k) if self.kv_fp8 else t(to_pool(self.k, "k").view(np.int16)),
            "v": t(self.v) if (self.v_int8 or self.kv_fp8) else
            t(to_pool(self.v, "v").view(np.int16)),
            "vs": t(self.vs) if (self.v_int8 or self.kv_fp8) else None,
            "err": torch.zeros(1, dtype=torch.int32, device=device),
        }
        return dev


def allclose_report(got, ref, atol=2e-3, rtol=1e-2):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = atol + rtol * np.abs(ref.astype(np.float64))
    bad = ~(err <= bound)
    return int(bad.sum()), float(np.nanmax(err)) if err.size else 0.0
