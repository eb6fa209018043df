"""GPU parity of the QKV projection with the append in its epilogue
(gkv_qkv_append).

Two contracts:
- qkv_out: x . W^T + bias against the oracle's orc_linear (run.cpp matmul +
  bias add, itself bit-exact with the reference's own code). bf16 products are
  exact and the sums are fp32 on the matrix cores, so the bound is in units of
  the sum of |products|: |gpu - ref| <= 2e-5 * sum_j |x_j w_ij| + 1e-6.
- the cache: every byte of the paged K and V (NaN-poisoned slots that must
  stay untouched included) equals what gkv_kv_append stores for the same
  qkv_out rows, and the stored K/V equal the oracle's orc_kv_append of those
  rows (bit-exact).
"""
import numpy as np
import pytest

from kvcase import INT8_POISON, from_pool

pytestmark = pytest.mark.gpu

D = 64
NAN16 = np.uint16(0x7FC1)


def bf16_round(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


class QkvCase:
    """rows of x (bf16 values), W, bias; a paged cache with a permuted table.
    Decode mode (prompts=None): row b is sequence b at position lens[b]-1.
    Prompt mode: rows are every position of each prompt (row_pos, row_seq)."""

    def __init__(self, seed, Hq, Hkv, hidden, lens=None, prompts=None, window=0, v_int8=False,
                 kv_fp8=False):
        rng = np.random.default_rng(seed)
        self.Hq, self.Hkv, self.hidden, self.window, self.v_int8 = Hq, Hkv, hidden, window, v_int8
        self.kv_fp8 = kv_fp8
        self.N = (Hq + 2 * Hkv) * D
        if prompts is None:
            self.lens = np.asarray(lens, np.int32)
            self.row_seq = np.arange(len(lens), dtype=np.int32)
            self.row_pos = self.lens - 1
            self.decode = True
        else:
            self.lens = np.asarray(prompts, np.int32)
            self.row_seq = np.concatenate([np.full(L, b, np.int32)
                                           for b, L in enumerate(prompts)]).astype(np.int32)
            self.row_pos = np.concatenate([np.arange(L, dtype=np.int32) for L in prompts])
            self.decode = False
        self.B = len(self.lens)
        self.M = len(self.row_pos)
        self.x = bf16_round(rng.standard_normal((self.M, hidden)))
        self.w = bf16_round(rng.standard_normal((self.N, hidden)) * 0.05)
        self.bias = (rng.standard_normal(self.N) * 0.1).astype(np.float32)
        # table: per sequence, blocks for all positions (full) or a ring of W slots
        if window:
            self.n_tbl = window // 16
        else:
            self.n_tbl = int((self.lens.max() + 15) // 16)
        self.NB = self.B * self.n_tbl + 3
        self.table = rng.permutation(self.NB)[:self.B * self.n_tbl].astype(np.int32).reshape(
            self.B, self.n_tbl)


def run(case, gkv, torch, dev, cache=True):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    x = t(case.x).to(torch.bfloat16)
    w = t(case.w).to(torch.bfloat16)
    cos, sin = gkv.rope_table(int(case.lens.max()) + 1)
    cos_d, sin_d = t(cos), t(sin)
    lens = t(case.lens)
    table = t(case.table)

    def new_cache():
        if case.kv_fp8:  # e4m3 codes poisoned with the NaN code, scales with NaN
            k = t(np.full((case.NB, case.Hkv, 16 * D), 0x7F, np.uint8))
            v = t(np.full((case.NB, case.Hkv, 16 * D), 0x7F, np.uint8))
            vs = t(np.full((case.NB, case.Hkv, 32), np.nan, np.float32))
            return k, v, vs, gkv.cache_view(k, v, table, case.Hkv, ring=case.window, v_scale=vs,
                                            v_format=gkv.KV_FP8)
        k = t(np.full((case.NB, case.Hkv, 16, D), NAN16, np.uint16).view(np.int16))
        vs = None
        if case.v_int8:
            v = t(np.full((case.NB, case.Hkv, 16 * D), INT8_POISON, np.int8))
            vs = t(np.full((case.NB, case.Hkv, 16), np.nan, np.float32))
        else:
            v = t(np.full((case.NB, case.Hkv, D, 16), NAN16, np.uint16).view(np.int16))
        view = gkv.cache_view(k, v, table, case.Hkv, ring=case.window, v_scale=vs)
        return k, v, vs, view

    qkv_out = torch.full((case.M, case.N), float("nan"), dtype=torch.float32, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    k1, v1, vs1, view1 = new_cache()
    row_pos = None if case.decode else t(case.row_pos)
    row_seq = None if case.decode else t(case.row_seq)
    gkv.qkv_append(x, w, t(case.bias), case.Hq, cos_d, sin_d, view1 if cache else None,
                   row_pos=row_pos, row_seq=row_seq, seq_lens=lens, qkv_out=qkv_out,
                   dev_err=err, n_kv_heads=case.Hkv)
    # the same rows through the plain append
    k2, v2, vs2, view2 = new_cache()
    if cache:
        gkv.kv_append(qkv_out, case.Hq, cos_d, sin_d, t(case.row_pos), view2,
                      row_seq=t(case.row_seq), seq_lens=lens)
    torch.cuda.synchronize()
    res = dict(err=int(err.item()), qkv=qkv_out.cpu().numpy(),
               k1=k1.cpu().numpy(), v1=v1.cpu().numpy(), k2=k2.cpu().numpy(),
               v2=v2.cpu().numpy(), cos=cos, sin=sin)
    if case.v_int8 or case.kv_fp8:
        res["vs1"], res["vs2"] = vs1.cpu().numpy(), vs2.cpu().numpy()
    return res


def check_projection(case, res, oracle, rows=None):
    """rows: the rows checked (default: all)."""
    rows = np.arange(case.M) if rows is None else np.asarray(rows)
    ref = oracle.linear(case.x[rows], case.w, case.bias)
    scale = np.abs(case.x[rows]).astype(np.float64) @ np.abs(case.w).astype(np.float64).T
    err = np.abs(res["qkv"][rows].astype(np.float64) - ref)
    bad = err > 2e-5 * scale + 1e-6
    assert not bad.any(), f"{int(bad.sum())} projections out of bound, max err {err.max()}"


def check_cache_fp8(case, res, oracle):
    """e4m3 K/V: every byte and scale equal to gkv_kv_append's, and the codes
    and scales of each stored row equal to the oracle's quantizer on the
    oracle's rotated key and on the value."""
    from kvcase import k_fp8_offsets, v_int8_offsets
    for a, b in (("k1", "k2"), ("v1", "v2")):
        assert np.array_equal(res[a], res[b]), f"{a} differs from gkv_kv_append's"
    assert np.array_equal(res["vs1"].view(np.uint32), res["vs2"].view(np.uint32)), "scales differ"
    _, k_rot, _, _ = oracle.kv_append(res["qkv"], case.Hq, case.Hkv, res["cos"], res["sin"],
                                      case.row_pos)
    v_rows = res["qkv"][:, (case.Hq + case.Hkv) * D:].reshape(case.M, case.Hkv, D)
    kc, ks = oracle.quantize_fp8(np.asarray(k_rot, np.float32).reshape(case.M, case.Hkv, D))
    vc, vsc = oracle.quantize_fp8(v_rows)
    n_checked = 0
    for r in range(case.M):
        b, p = int(case.row_seq[r]), int(case.row_pos[r])
        if case.window and p + case.window < case.lens[b]:
            continue
        slot = p % case.window if case.window else p
        phys, off = case.table[b, slot // 16], slot % 16
        assert np.array_equal(res["k1"][phys][:, k_fp8_offsets(off)], kc[r]), f"K of row {r}"
        assert np.array_equal(res["v1"][phys][:, v_int8_offsets(off)], vc[r]), f"V of row {r}"
        assert np.array_equal(res["vs1"][phys, :, off].view(np.uint32), ks[r].view(np.uint32))
        assert np.array_equal(res["vs1"][phys, :, 16 + off].view(np.uint32),
                              vsc[r].view(np.uint32))
        n_checked += 1
    assert n_checked > 0


def check_cache(case, res, oracle):
    if case.kv_fp8:
        return check_cache_fp8(case, res, oracle)
    assert np.array_equal(res["k1"], res["k2"]), "K cache bytes differ from gkv_kv_append's"
    assert np.array_equal(res["v1"], res["v2"]), "V cache bytes differ from gkv_kv_append's"
    if case.v_int8:
        assert np.array_equal(res["vs1"].view(np.uint32), res["vs2"].view(np.uint32)), \
            "V scales differ"
    # the stored K/V against the oracle's append of the same qkv rows (rows
    # whose ring slot a later row takes are skipped)
    _, _, kb, vb = oracle.kv_append(res["qkv"], case.Hq, case.Hkv, res["cos"], res["sin"],
                                    case.row_pos)
    kl = from_pool(res["k1"].view(np.uint16), "k")
    vl = None if case.v_int8 else from_pool(res["v1"].view(np.uint16), "v")
    n_checked = 0
    for r in range(case.M):
        b, p = int(case.row_seq[r]), int(case.row_pos[r])
        if case.window and p + case.window < case.lens[b]:
            continue
        slot = p % case.window if case.window else p
        phys, off = case.table[b, slot // 16], slot % 16
        assert np.array_equal(kl[phys, :, off, :], kb[r]), f"K of row {r}"
        if vl is not None:
            assert np.array_equal(vl[phys, :, :, off], vb[r]), f"V of row {r}"
        n_checked += 1
    assert n_checked > 0


def test_decode_config2_shape(oracle, gkv, cuda):
    import torch
    rng = np.random.default_rng(2)
    lens = rng.integers(128, 2049, 512)
    case = QkvCase(3, 64, 8, 2880, lens=lens)
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


def test_decode_window_ring(oracle, gkv, cuda):
    import torch
    rng = np.random.default_rng(5)
    lens = rng.integers(1, 4097, 96)
    case = QkvCase(6, 64, 8, 576, lens=lens, window=128)
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


@pytest.mark.parametrize("window", [0, 128])
def test_prompt_rows(oracle, gkv, cuda, window):
    import torch
    case = QkvCase(11 + window, 8, 2, 256, prompts=[300, 17, 129, 1, 64], window=window)
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


def test_int8_v(oracle, gkv, cuda):
    import torch
    rng = np.random.default_rng(8)
    case = QkvCase(9, 16, 4, 512, lens=rng.integers(1, 300, 100), v_int8=True)
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


def test_fp8_kv(oracle, gkv, cuda):
    """The e4m3 K/V cache from the projection's epilogue: decode rows on a full
    layer and prompt rows (the 128 x 128 tiles) on a ring."""
    import torch
    rng = np.random.default_rng(31)
    for case in (QkvCase(32, 16, 4, 512, lens=rng.integers(1, 300, 100), kv_fp8=True),
                 QkvCase(33, 64, 8, 2880, prompts=[900, 700, 500], window=128, kv_fp8=True)):
        res = run(case, gkv, torch, cuda)
        assert res["err"] == 0
        check_cache(case, res, oracle)


@pytest.mark.parametrize("hidden", [64, 128, 192])
def test_short_hidden(oracle, gkv, cuda, hidden):
    """Fewer than three K chunks: the row placement finishes after the loop."""
    import torch
    rng = np.random.default_rng(hidden)
    case = QkvCase(hidden, 8, 2, hidden, lens=rng.integers(1, 100, 70))
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


def test_odd_head_count_and_ragged_rows(oracle, gkv, cuda):
    """7 heads (the last column block half used) and 77 rows (a partial row block)."""
    import torch
    rng = np.random.default_rng(12)
    case = QkvCase(13, 5, 1, 320, lens=rng.integers(1, 80, 77))
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


def test_many_rows_large_tiles(oracle, gkv, cuda):
    """2,000+ rows take the 128 x 128 tiles: prompt rows with a ragged last
    row block and a ring window."""
    import torch
    case = QkvCase(16, 8, 2, 256, prompts=[700, 513, 900, 1], window=128)
    assert case.M >= 2048
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    check_projection(case, res, oracle)
    check_cache(case, res, oracle)


@pytest.mark.parametrize("v_int8", [False, True])
def test_gpt_oss_shape_large_tiles(oracle, gkv, cuda, v_int8):
    """A prompt batch of the gpt-oss shape (Hq 64, Hkv 8, hidden 2880, N 5120)
    past 2,048 rows: the 128 x 128 tiles with their 40 column blocks spread
    over the XCDs, a ragged last row block, bf16 and int8 V. Every cache byte
    is checked; the projection on 300 sampled rows and every row of the last
    row block."""
    import torch
    case = QkvCase(17 + int(v_int8), 64, 8, 2880, prompts=[800, 640, 512, 130], v_int8=v_int8)
    assert case.M >= 2048 and case.M % 128 != 0
    res = run(case, gkv, torch, cuda)
    assert res["err"] == 0
    rng = np.random.default_rng(3)
    rows = np.unique(np.concatenate([rng.choice(case.M, 300, replace=False),
                                     np.arange(case.M // 128 * 128, case.M)]))
    check_projection(case, res, oracle, rows)
    check_cache(case, res, oracle)


def test_projection_only(oracle, gkv, cuda):
    import torch
    case = QkvCase(14, 64, 8, 2880, lens=np.full(33, 5))
    res = run(case, gkv, torch, cuda, cache=False)
    check_projection(case, res, oracle)
    assert np.array_equal(res["k1"], res["k2"]) and np.array_equal(res["v1"], res["v2"])


def test_bad_block_id_flagged(gkv, cuda):
    """A table entry outside the pool: the row is not stored, the error word
    gets GKV_DEVERR_BLOCK_ID, nothing faults."""
    import torch
    case = QkvCase(15, 8, 2, 128, lens=np.array([20, 40, 3]))
    case.table[1, 2] = case.NB + 100  # row 1 sits at position 39: block 2
    res = run(case, gkv, torch, cuda)
    assert res["err"] & 1
    poison = np.full_like(res["k1"], np.int16(np.uint16(0x7FC1).view(np.int16)))
    assert np.array_equal(res["k1"], res["k2"])
    assert not np.array_equal(res["k1"], poison)
