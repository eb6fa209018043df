"""GPU parity of chunked prefill over a paged history (gkv_prefill_paged).

Each prompt is fed in two chunks. Chunk 1 (positions 0 .. C-1, C a multiple
of 16) is appended into the paged cache and attended to with start 0; chunk 2
(positions C .. L-1) attends to the history C tokens from the cache and to
itself. Every output row is compared with the one-shot oracle prefill of the
whole prompt (orc_prefill_attention: the reference's decode attention at
every position, run.cpp:597-642) within max-abs 2e-3 + rel 1e-2.

- Full layer, chunk 2's keys from its packed rows (history from the cache).
- Full layer, chunk 2 appended first and every key from the cache (also the
  load slots past the block's last tile: they re-read cached blocks).
- Ring layer (window 128): chunk 2 attended before it is appended (the ring
  still holds the last 128 positions of chunk 1), then appended.
- The same three on the int8-V cache (the reference engine's format) and on
  the e4m3 K/V cache: the keys read from the cache stand for what the cache
  holds (int8: code * scale, orc_quantize_v of the fp32 V, pinned to the
  reference's quantize_v; e4m3: value(code) * scale of the rotated K and of
  V, orc_quantize_fp8), those from packed rows for their bf16 values.
- Error words: a start that is not a multiple of 16, and a V beyond the
  prefill's range (bf16 and int8 V); small V (|v| ~ 1e-2 and 2^-20) within
  the tolerance.
"""
import numpy as np
import pytest

from kvcase import allclose_report

pytestmark = pytest.mark.gpu

D = 64


class Chunked:
    def __init__(self, torch, gkv, oracle, L, C, Hq=64, Hkv=8, window=0, seed=0, scale=0.5,
                 fmt="bf16"):
        rng = np.random.default_rng(seed)
        self.torch, self.gkv = torch, gkv
        self.L = np.asarray(L, np.int32)
        self.C = np.asarray(C, np.int32)
        assert np.all(self.C % 16 == 0) and np.all(self.C <= self.L)
        self.B, self.Hq, self.Hkv, self.window = len(L), Hq, Hkv, window
        cu = np.concatenate([[0], np.cumsum(self.L)]).astype(np.int32)
        T = int(cu[-1])
        self.qkv = (rng.standard_normal((T, (Hq + 2 * Hkv) * D)) * scale).astype(np.float32)
        self.sinks = rng.standard_normal(Hq).astype(np.float32)
        pos = np.concatenate([np.arange(n) for n in self.L]).astype(np.int32)
        cos, sin = oracle.rope_table(int(self.L.max()))
        self.oracle, self.cu_all, self.pos, self.cos, self.sin = oracle, cu, pos, cos, sin
        k_rot = self.reference()
        # what a quantized cache stands for: the fp32 (rotated K and) V quantized per
        # token and head
        self.fmt = fmt
        v32 = self.qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D)
        self.k_q, self.v_q = self.k_f, self.v_bf
        if fmt == "int8":
            self.v_q = oracle.dequantize_v(*oracle.quantize_v(v32))
        elif fmt == "fp8":
            self.k_q = oracle.dequantize_fp8(*oracle.quantize_fp8(k_rot.reshape(T, Hkv, D)))
            self.v_q = oracle.dequantize_fp8(*oracle.quantize_fp8(v32))
        # the pool: one layer (a ring layer when window > 0), NaN in every slot
        self.pool = gkv.Pool(n_layers=1, n_kv_heads=Hkv, max_seqs=self.B,
                             max_seq_len=int(self.L.max()), window=window,
                             num_blocks=int(((self.L + 15) // 16).sum()) + 8,
                             shuffle_seed=seed + 3,
                             v_format={"bf16": gkv.V_BF16, "int8": gkv.V_INT8,
                                       "fp8": gkv.KV_FP8}[fmt])
        for b in range(self.B):
            assert self.pool.seq_alloc() == b
            assert self.pool.reserve(b, int(self.L[b])) == 0
        self.pool.sync()
        self.view = self.pool.view(0)
        n = self.view.num_blocks * Hkv * 16 * D
        nan = torch.full((n,), -1, dtype=torch.int16, device="cuda")  # bf16 0xffff: NaN
        # codes 0xff (int8 -1, e4m3 NaN), scales NaN (fp32 0xffffffff)
        gkv.hip_memcpy_d2d(self.view.k, nan.data_ptr(), n if fmt == "fp8" else n * 2)
        gkv.hip_memcpy_d2d(self.view.v, nan.data_ptr(), n if fmt != "bf16" else n * 2)
        if fmt != "bf16":
            gkv.hip_memcpy_d2d(self.view.v_scale, nan.data_ptr(),
                               n // D * (8 if fmt == "fp8" else 4))
        torch.cuda.synchronize()
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to("cuda")  # noqa: E731
        self.t = t
        self.cos_d, self.sin_d = t(cos), t(sin)
        self.sinks_d = t(self.sinks)

    def reference(self):
        """The oracle's prefill of the whole prompts from the current qkv rows
        (call again after changing them); returns the rotated fp32 keys."""
        o = self.oracle
        q_rot, k_rot, kb, vb = o.kv_append(self.qkv, self.Hq, self.Hkv, self.cos, self.sin,
                                           self.pos)
        self.q_rot, self.k_f, self.v_bf = q_rot, o.from_bf16(kb), o.from_bf16(vb)
        self.ref = o.prefill_attention(self.cu_all, q_rot, self.k_f, self.v_bf, self.sinks,
                                       window=self.window)
        return k_rot

    def chunk_rows(self, which):
        """Rows (indices into the whole-prompt arrays) of chunk 1 or 2, prompt by prompt."""
        rows, cu = [], [0]
        for b in range(self.B):
            lo, hi = (0, self.C[b]) if which == 1 else (self.C[b], self.L[b])
            rows.append(np.arange(self.cu_all[b] + lo, self.cu_all[b] + hi))
            cu.append(cu[-1] + hi - lo)
        return np.concatenate(rows).astype(np.int64), np.asarray(cu, np.int32)

    def append(self, which, err):
        """The chunk's rows into the cache; the lengths after it (C or L) tell
        a ring which rows it keeps."""
        rows, cu = self.chunk_rows(which)
        seq = np.repeat(np.arange(self.B), np.diff(cu)).astype(np.int32)
        lens = self.C if which == 1 else self.L
        self.gkv.kv_append(self.t(self.qkv[rows]), self.Hq, self.cos_d, self.sin_d,
                           self.t(self.pos[rows]), self.view, row_seq=self.t(seq),
                           seq_lens=self.t(lens), dev_err=err)

    def packed(self, which):
        """The chunk's packed bf16 K/V rows (gkv_kv_append with no cache)."""
        torch = self.torch
        rows, _ = self.chunk_rows(which)
        n = max(len(rows), 1)
        kp = torch.zeros((n, self.Hkv * D), dtype=torch.int16, device="cuda")
        vp = torch.zeros((n, self.Hkv * D), dtype=torch.int16, device="cuda")
        none = self.gkv.CacheView(None, None, None, 0, 0, self.Hkv, 0)
        self.gkv.kv_append(self.t(self.qkv[rows]), self.Hq, self.cos_d, self.sin_d,
                           self.t(self.pos[rows]), none, k_pack=kp, v_pack=vp)
        return kp, vp

    def prefill(self, which, err, k=None, v=None, start=None):
        torch = self.torch
        rows, cu = self.chunk_rows(which)
        if start is None:
            start = np.zeros(self.B, np.int32) if which == 1 else self.C
        out = torch.full((max(len(rows), 1), self.Hq * D), float("nan"), dtype=torch.float32,
                         device="cuda")
        self.gkv.prefill_paged(self.t(cu), int(np.diff(cu).max()), self.t(self.qkv[rows]),
                               self.view, self.sinks_d, out, start_pos=self.t(start.astype(np.int32)),
                               k=k, v=v, window=self.window, cos_tab=self.cos_d,
                               sin_tab=self.sin_d, dev_err=err)
        torch.cuda.synchronize()
        return out.cpu().numpy()[:len(rows)].reshape(len(rows), self.Hq, D), rows

    def ref_with_cache(self, rows, n_cached):
        """The oracle's rows when the first n_cached[b] positions of prompt b
        are read from a quantized cache (the rest from packed bf16 rows)."""
        k, v = self.k_f.copy(), self.v_bf.copy()
        for b in range(self.B):
            lo = self.cu_all[b]
            k[lo:lo + n_cached[b]] = self.k_q[lo:lo + n_cached[b]]
            v[lo:lo + n_cached[b]] = self.v_q[lo:lo + n_cached[b]]
        return self.oracle.prefill_attention(self.cu_all, self.q_rot, k, v, self.sinks,
                                             window=self.window)[rows]

    def check(self, got, rows, what, n_cached=None):
        want = self.ref[rows] if n_cached is None or self.fmt == "bf16" else \
            self.ref_with_cache(rows, n_cached)
        if self.fmt == "fp8" and n_cached is not None:
            # the e4m3 cache moves the output beyond the tolerance: the
            # comparison tells the formats apart
            assert allclose_report(want, self.ref[rows])[0] > 0
        bad, worst = allclose_report(got, want)
        assert bad == 0, f"{what}: {bad} outputs out of tolerance (max err {worst:.3e})"
        return worst


LENS = [300, 517, 64, 130, 1040, 33]
CUTS = [128, 256, 48, 128, 512, 16]


@pytest.mark.parametrize("fmt", ["bf16", "int8", "fp8"])
@pytest.mark.parametrize("cache_only", [False, True])
def test_two_chunks_full_layer(oracle, gkv, cuda, cache_only, fmt):
    import torch
    c = Chunked(torch, gkv, oracle, LENS, CUTS, seed=11, fmt=fmt)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        kp, vp = c.packed(1)
        c.append(1, err)
        got, rows = c.prefill(1, err, k=kp, v=vp)
        w1 = c.check(got, rows, "chunk 1")
        if cache_only:
            c.append(2, err)                      # chunk 2 into the cache first
            got, rows = c.prefill(2, err)         # every key from the cache
        else:
            kp, vp = c.packed(2)
            got, rows = c.prefill(2, err, k=kp, v=vp)  # history from the cache
            c.append(2, err)
        w2 = c.check(got, rows, "chunk 2", n_cached=c.L if cache_only else c.C)
        assert int(err.item()) == 0
        print(f"full layer cache_only={cache_only} {fmt}: max abs err "
              f"{w1:.2e} / {w2:.2e}")
    finally:
        c.pool.close()


@pytest.mark.parametrize("fmt", ["bf16", "int8", "fp8"])
@pytest.mark.parametrize("window", [128, 32])
def test_two_chunks_ring_layer(oracle, gkv, cuda, fmt, window):
    """Window W on a ring of W slots: chunk 2 attends to the ring's history
    before its own append overwrites it."""
    import torch
    c = Chunked(torch, gkv, oracle, [400, 700, 96, 260], [256, 512, 32, 128], window=window,
                seed=12 + window, fmt=fmt)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        kp, vp = c.packed(1)
        got, rows = c.prefill(1, err, k=kp, v=vp)
        c.append(1, err)
        c.check(got, rows, "chunk 1")
        kp, vp = c.packed(2)
        got, rows = c.prefill(2, err, k=kp, v=vp)
        c.append(2, err)
        c.check(got, rows, "chunk 2", n_cached=c.C)
        assert int(err.item()) == 0
    finally:
        c.pool.close()


@pytest.mark.parametrize("fmt", ["bf16", "int8", "fp8"])
@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (8, 4), (8, 8), (12, 2)])
def test_group_sizes(oracle, gkv, cuda, Hq, Hkv, fmt):
    """Groups of 4, 2, 1 and 6 query heads per kv head (the 4-, 2- and 1-wave
    and a partly idle 8-wave workgroup of the history kernel), every cache
    format: chunk 2 from packed rows over a cached history, then a full
    re-read of both chunks from the cache."""
    import torch
    c = Chunked(torch, gkv, oracle, [150, 97, 33], [64, 80, 16], Hq=Hq, Hkv=Hkv,
                seed=Hq * 10 + Hkv, fmt=fmt)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        c.append(1, err)
        kp, vp = c.packed(2)
        got, rows = c.prefill(2, err, k=kp, v=vp)
        c.check(got, rows, "chunk 2 over the cached history", n_cached=c.C)
        c.append(2, err)
        got, rows = c.prefill(2, err)
        c.check(got, rows, "chunk 2 from the cache", n_cached=c.L)
        assert int(err.item()) == 0
    finally:
        c.pool.close()


def test_start_not_a_block_multiple_is_flagged(oracle, gkv, cuda):
    import torch
    c = Chunked(torch, gkv, oracle, [100, 80], [32, 48], seed=13)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        c.append(1, err)
        kp, vp = c.packed(2)
        got, _ = c.prefill(2, err, k=kp, v=vp, start=np.array([32, 40], np.int32))
        assert int(err.item()) & gkv.DEVERR_ALIGN
        assert np.isfinite(got).all()
    finally:
        c.pool.close()


def test_start_not_a_block_multiple_is_flagged_cache_only(oracle, gkv, cuda):
    """The same with every key from the cache (k = v = NULL, both chunks
    appended first): the misaligned prompt's outputs are meaningless but
    finite, and the error bit is set."""
    import torch
    c = Chunked(torch, gkv, oracle, [100, 80], [32, 48], seed=14)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        c.append(1, err)
        c.append(2, err)
        got, _ = c.prefill(2, err, start=np.array([32, 40], np.int32))
        assert int(err.item()) & gkv.DEVERR_ALIGN
        assert np.isfinite(got).all()
    finally:
        c.pool.close()


@pytest.mark.parametrize("cache_only", [False, True])
def test_history_block_outside_the_pool_is_flagged(oracle, gkv, cuda, cache_only):
    """A history block id outside the pool (one table entry overwritten after
    the first chunk went in): the history prefill flags GKV_DEVERR_BLOCK_ID
    and reads block 0 instead of faulting; every output stays finite, and the
    prompts whose tables are intact still match the oracle."""
    import torch
    c = Chunked(torch, gkv, oracle, [160, 96, 130], [96, 64, 80], seed=15)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    try:
        c.append(1, err)
        if cache_only:
            c.append(2, err)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        # prompt 0's second history block -> an id past the pool
        bad = torch.tensor([c.view.num_blocks + 5], dtype=torch.int32, device="cuda")
        gkv.hip_memcpy_d2d(c.view.block_table + 4 * 1, bad.data_ptr(), 4)
        torch.cuda.synchronize()
        kp, vp = (None, None) if cache_only else c.packed(2)
        got, rows = c.prefill(2, err, k=kp, v=vp)
        assert int(err.item()) & gkv.DEVERR_BLOCK_ID
        assert np.isfinite(got).all()
        # prompts 1 and 2 did not use the bad entry
        _, cu = c.chunk_rows(2)
        keep = np.arange(cu[1], cu[3])
        c.check(got[keep], rows[keep], "intact prompts")
    finally:
        c.pool.close()


def test_v_beyond_range_is_flagged(oracle, gkv, cuda):
    """|v| >= 2^26 leaves the fp16 range of the staged v * 2^-10: the error
    word says so (the output holds inf there), on the bf16 and on the int8-V
    cache."""
    import torch
    for fmt in ("bf16", "int8"):
        c = Chunked(torch, gkv, oracle, [64], [32], seed=14, fmt=fmt)
        Hq, Hkv = c.Hq, c.Hkv
        c.qkv[40, (Hq + Hkv) * D + 5] = 2.0 ** 27  # chunk 2, V of kv head 0, dim 5
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        try:
            c.append(1, err)
            kp, vp = c.packed(2)
            c.prefill(2, err, k=kp, v=vp)
            assert int(err.item()) & gkv.DEVERR_RANGE, fmt
        finally:
            c.pool.close()


def test_small_v_within_tolerance(oracle, gkv, cuda):
    """Below the staged range (|v| < 2^-4, fp16 of v * 2^-10 subnormal) the
    error stays within 2^-15 absolute: values of 2^-20 and 3e-3 in the cached
    history and in the chunk are attended within the tolerance, with no error
    word."""
    import torch
    c = Chunked(torch, gkv, oracle, [100, 70], [48, 32], seed=15, scale=0.01)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    Hq, Hkv = c.Hq, c.Hkv
    v0 = (Hq + Hkv) * D
    c.qkv[60, v0 + 9] = 2.0 ** -20
    c.reference()
    try:
        c.append(1, err)
        kp, vp = c.packed(2)
        got, rows = c.prefill(2, err, k=kp, v=vp)
        assert int(err.item()) == 0
        c.check(got, rows, "small V")
    finally:
        c.pool.close()
