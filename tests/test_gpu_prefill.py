"""GPU parity of the prefill path against the CPU oracle.

A batch of prompts is appended in one gkv_kv_append call (every row of every
prompt, into an empty paged cache with a permuted block table), which must be
bit-exact: the rotated Q, the packed bf16 K/V rows and every byte of the cache
(NaN-poisoned slots that must stay untouched included; on a ring layer only the
last W positions of each prompt are stored). Then gkv_prefill_attention on the
packed rows is compared with orc_prefill_attention -- the reference's decode
attention (run.cpp:597-642) at every prompt position -- within max-abs 2e-3 +
rel 1e-2 (bf16 K/V, fp32 accumulate).
"""
import numpy as np
import pytest

from kvcase import INT8_POISON, allclose_report, from_pool, v_int8_offsets

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
D = 64
NAN16 = np.uint16(0x7FC1)


class PrefillCase:
    def __init__(self, oracle, seed, lengths, Hq, Hkv, window=0, scale=0.5, sink_scale=1.0,
                 v_int8=False):
        rng = np.random.default_rng(seed)
        self.v_int8 = v_int8
        self.L = np.asarray(lengths, np.int64)
        self.B = len(self.L)
        self.Hq, self.Hkv, self.window = Hq, Hkv, window
        self.cu = np.concatenate([[0], np.cumsum(self.L)]).astype(np.int32)
        T = int(self.cu[-1])
        self.T = T
        self.qkv = (rng.standard_normal((T, (Hq + 2 * Hkv) * D)) * scale).astype(np.float32)
        self.sinks = (rng.standard_normal(Hq) * sink_scale).astype(np.float32)
        self.pos = np.concatenate([np.arange(l) for l in self.L]).astype(np.int32)
        self.row_seq = np.repeat(np.arange(self.B), self.L).astype(np.int32)
        self.max_len = int(self.L.max()) if self.B else 0
        self.cos, self.sin = oracle.rope_table(max(self.max_len, 1))
        self.q_rot, _, self.kb, self.vb = oracle.kv_append(self.qkv, Hq, Hkv, self.cos,
                                                           self.sin, self.pos)
        # paged cache: per sequence, blocks for all positions (full) or a ring of W slots
        slots = [min(int(l), window) if window else int(l) for l in self.L]
        self.n_tbl = max([(window // 16) if window else (int(l) + 15) // 16 for l in self.L] + [1])
        nb_need = sum((s + 15) // 16 for s in slots) if not window else self.B * (window // 16)
        self.NB = nb_need + 5
        perm = rng.permutation(self.NB)
        self.table = np.full((self.B, self.n_tbl), -1, np.int32)
        i = 0
        for b in range(self.B):
            nb = (window // 16) if window else (int(self.L[b]) + 15) // 16
            self.table[b, :nb] = perm[i:i + nb]
            i += nb
        self.k_expect = np.full((self.NB, Hkv, 16, D), NAN16, np.uint16)
        if v_int8:
            self.v_expect = np.full((self.NB, Hkv, 16 * D), INT8_POISON, np.int8)
            self.vs_expect = np.full((self.NB, Hkv, 16), np.nan, np.float32)
            v_rows = self.qkv[:, (Hq + Hkv) * D:].reshape(T, Hkv, D)
            codes, scales = oracle.quantize_v(v_rows)
        else:
            self.v_expect = np.full((self.NB, Hkv, D, 16), NAN16, np.uint16)
        for r in range(T):
            b, p = int(self.row_seq[r]), int(self.pos[r])
            if window and p + window < self.L[b]:
                continue  # overwritten later in the ring
            slot = p % window if window else p
            blk, off = self.table[b, slot // 16], slot % 16
            self.k_expect[blk, :, off, :] = self.kb[r]
            if v_int8:
                self.v_expect[blk][:, v_int8_offsets(off)] = codes[r]
                self.vs_expect[blk, :, off] = scales[r]
            else:
                self.v_expect[blk, :, :, off] = self.vb[r]

    def oracle_out(self):
        from oracle import kv_oracle as O
        return O.prefill_attention(self.cu, self.q_rot, O.from_bf16(self.kb),
                                   O.from_bf16(self.vb), self.sinks, window=self.window)


def run_gpu(case, gkv, torch, dev, out_dtype=None, ring=True, rotate_in_prefill=False):
    """rotate_in_prefill: the append writes no rotated Q; the prefill reads
    the qkv rows and rotates Q on load."""
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    qkv = t(case.qkv)
    cos, sin = gkv.rope_table(max(case.max_len, 1))
    k = t(np.full((case.NB, case.Hkv, 16, D), NAN16, np.uint16).view(np.int16))
    vs = None
    if case.v_int8:
        v = t(np.full((case.NB, case.Hkv, 16 * D), INT8_POISON, np.int8))
        vs = t(np.full((case.NB, case.Hkv, 16), np.nan, np.float32))
    else:
        v = t(np.full((case.NB, case.Hkv, D, 16), NAN16, np.uint16).view(np.int16))
    table = t(case.table)
    view = gkv.cache_view(k, v, table, case.Hkv, ring=case.window if ring else 0, v_scale=vs)
    T = max(case.T, 1)
    q_out = torch.full((T, case.Hq * D), float("nan"), dtype=torch.float32, device=dev)
    k_pack = torch.zeros((T, case.Hkv * D), dtype=torch.int16, device=dev)
    v_pack = torch.zeros((T, case.Hkv * D), dtype=torch.int16, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    lens = t(case.L.astype(np.int32))
    cos_d, sin_d = t(cos), t(sin)
    gkv.kv_append(qkv, case.Hq, cos_d, sin_d, t(case.pos), view, row_seq=t(case.row_seq),
                  seq_lens=lens, q_out=None if rotate_in_prefill else q_out, k_pack=k_pack,
                  v_pack=v_pack, dev_err=err)
    out = torch.full((T, case.Hq * D), float("nan"), dtype=out_dtype or torch.float32,
                     device=dev)
    if rotate_in_prefill:
        gkv.prefill_attention(t(case.cu), case.max_len, qkv, k_pack, v_pack, t(case.sinks), out,
                              case.Hkv, window=case.window, cos_tab=cos_d, sin_tab=sin_d)
    else:
        gkv.prefill_attention(t(case.cu), case.max_len, q_out, k_pack, v_pack, t(case.sinks),
                              out, case.Hkv, window=case.window)
    torch.cuda.synchronize()
    return dict(
        err=int(err.item()),
        q=q_out.cpu().numpy()[:case.T].reshape(case.T, case.Hq, D),
        kp=k_pack.cpu().numpy().view(np.uint16)[:case.T].reshape(case.T, case.Hkv, D),
        vp=v_pack.cpu().numpy().view(np.uint16)[:case.T].reshape(case.T, case.Hkv, D),
        k=from_pool(k.cpu().numpy().view(np.uint16), "k"),
        v=v.cpu().numpy() if case.v_int8 else from_pool(v.cpu().numpy().view(np.uint16), "v"),
        vs=vs.cpu().numpy() if case.v_int8 else None,
        out=out.float().cpu().numpy()[:case.T].reshape(case.T, case.Hq, D))


def check(case, res, atol=ATOL, rtol=RTOL):
    assert res["err"] == 0
    assert np.array_equal(res["q"].view(np.uint32), case.q_rot.view(np.uint32)), "rotated Q bits"
    assert np.array_equal(res["kp"], case.kb), "packed K bits"
    assert np.array_equal(res["vp"], case.vb), "packed V bits"
    assert np.array_equal(res["k"], case.k_expect), "K cache bytes differ"
    assert np.array_equal(res["v"], case.v_expect), "V cache bytes differ"
    if case.v_int8:
        assert np.array_equal(res["vs"].view(np.uint32), case.vs_expect.view(np.uint32)), \
            "V scales differ"
    ref = case.oracle_out()
    n_bad, max_err = allclose_report(res["out"], ref, atol, rtol)
    assert n_bad == 0, f"{n_bad} outputs outside tolerance, max abs err {max_err}"


@pytest.mark.parametrize("window", [0, 128])
def test_config4_shape(oracle, gkv, cuda, window):
    import torch
    rng = np.random.default_rng(40 + window)
    lengths = rng.integers(64, 513, size=16)
    case = PrefillCase(oracle, 41 + window, lengths, 64, 8, window=window)
    check(case, run_gpu(case, gkv, torch, cuda))


@pytest.mark.parametrize("window", [0, 128])
def test_config4_full_batch(oracle, gkv, cuda, window):
    """Config 4 at its benchmark size: 64 prompts of U[64, 512] tokens (about
    18k rows, 5,000+ workgroups), every output row against the oracle."""
    import torch
    rng = np.random.default_rng(400 + window)
    lengths = rng.integers(64, 513, size=64)
    case = PrefillCase(oracle, 401 + window, lengths, 64, 8, window=window)
    check(case, run_gpu(case, gkv, torch, cuda))


@pytest.mark.parametrize("window", [0, 16, 128])
def test_edge_lengths(oracle, gkv, cuda, window):
    import torch
    lengths = [1, 2, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 200]
    case = PrefillCase(oracle, 7 + window, lengths, 64, 8, window=window)
    check(case, run_gpu(case, gkv, torch, cuda))


@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (8, 8), (8, 4), (12, 2)])
def test_group_sizes(oracle, gkv, cuda, Hq, Hkv):
    """Config 1 shape (group 4) and groups 1, 2, 6 (6 waves of an 8-wave workgroup)."""
    import torch
    lengths = [1, 37, 100, 256]
    case = PrefillCase(oracle, Hq * 10 + Hkv, lengths, Hq, Hkv, window=0)
    check(case, run_gpu(case, gkv, torch, cuda))


@pytest.mark.parametrize("window", [0, 128])
def test_long_prompts(oracle, gkv, cuda, window):
    """Prompts of 1,000-2,000 rows: 16-32 key tiles per query block, so the
    4-stage K/V tile pipeline wraps many times (and its past-the-end loads
    re-read the last rows)."""
    import torch
    case = PrefillCase(oracle, 60 + window, [2000, 1031, 64], 64, 8, window=window)
    check(case, run_gpu(case, gkv, torch, cuda))


def test_large_scores_bf16_out(oracle, gkv, cuda):
    """Scores spread over tens of units (peaked softmax, rescales), bf16 output."""
    import torch
    case = PrefillCase(oracle, 99, [90, 300, 5], 64, 8, window=0, scale=2.0, sink_scale=4.0)
    res = run_gpu(case, gkv, torch, cuda, out_dtype=torch.bfloat16)
    ref = case.oracle_out()
    n_bad, max_err = allclose_report(res["out"], ref, ATOL, RTOL + 2 ** -8)  # + bf16 output rounding
    assert n_bad == 0, f"{n_bad} outputs outside tolerance, max abs err {max_err}"


@pytest.mark.parametrize("window", [0, 128])
def test_prompt_append_into_int8_v_cache(oracle, gkv, cuda, window):
    """Whole prompts appended into an int8-V cache: codes and scales of every
    stored row bit-exact (ring: the last W positions), packed K/V unchanged."""
    import torch
    case = PrefillCase(oracle, 90 + window, [1, 16, 130, 300], 64, 8, window=window,
                       v_int8=True)
    check(case, run_gpu(case, gkv, torch, cuda))


@pytest.mark.parametrize("window", [0, 128])
def test_rotate_on_load_matches_rotated_q(oracle, gkv, cuda, window):
    """The prefill rotating Q from the raw qkv rows gives the same output bits
    as the prefill on the append's rotated Q (and matches the oracle)."""
    import torch
    case = PrefillCase(oracle, 95 + window, [1, 33, 130, 300, 517], 64, 8, window=window)
    a = run_gpu(case, gkv, torch, cuda)
    b = run_gpu(case, gkv, torch, cuda, rotate_in_prefill=True)
    check(case, a)
    assert np.array_equal(a["out"].view(np.uint32), b["out"].view(np.uint32))


def test_empty_batch_and_zero_length(oracle, gkv, cuda):
    import torch
    case = PrefillCase(oracle, 5, [0, 20, 0, 33], 64, 8, window=128)
    check(case, run_gpu(case, gkv, torch, cuda))
    # B = 0 is a no-op
    out = torch.zeros(1, 64 * 64, device=cuda)
    z = torch.zeros(1, dtype=torch.int32, device=cuda)
    q = torch.zeros(1, 64 * 64, device=cuda)
    kv = torch.zeros(1, 8 * 64, dtype=torch.int16, device=cuda)
    gkv.prefill_attention(z, 0, q, kv, kv, torch.zeros(64, device=cuda), out, 8)
    torch.cuda.synchronize()
    assert float(out.abs().sum()) == 0.0


def _sweep_draw(seed):
    rng = np.random.default_rng(9100 + seed)
    Hkv = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.choice([1, 2, 3, 4, 6, 8]))
    B = int(rng.integers(1, 25))
    kind = str(rng.choice(["short", "mixed", "long"]))
    if kind == "short":
        L = rng.integers(0, 48, size=B)
    elif kind == "mixed":
        L = np.where(rng.random(B) < 0.15, 0, rng.integers(1, 600, size=B))
    else:
        L = rng.integers(300, 900, size=B)
    # at most ~4000 prompt rows, so the oracle finishes in seconds
    L = L[:max(1, int(np.searchsorted(np.cumsum(L), 4000)))]
    window = int(rng.choice([0, 0, 16, 32, 128]))
    return dict(Hq=Hkv * G, Hkv=Hkv, L=L, window=window, rot=bool(rng.random() < 0.5),
                bf16=bool(rng.random() < 0.3), scale=float(rng.choice([0.5, 1.0, 2.0])),
                seed=9200 + seed)


@pytest.mark.parametrize("seed", range(24))
def test_prefill_sweep(oracle, gkv, cuda, seed):
    """Seeded shapes: kv heads 1-8, 1-8 query heads per kv head, 1-24 prompts
    of 0 to 900 tokens, windows 0/16/32/128, Q rotated by the append or on
    load, fp32 or bf16 output, value scales 0.5-2. The append is bit-exact
    (rotated Q when the append writes it, packed rows, cache bytes) and the
    output within max-abs 2e-3 + rel 1e-2 (plus bf16 rounding)."""
    import torch
    p = _sweep_draw(seed)
    print(f"prefill sweep {seed}: Hq={p['Hq']} Hkv={p['Hkv']} B={len(p['L'])} "
          f"rows={int(p['L'].sum())} W={p['window']} rot={p['rot']} bf16={p['bf16']}",
          flush=True)
    case = PrefillCase(oracle, p["seed"], p["L"], p["Hq"], p["Hkv"], window=p["window"],
                       scale=p["scale"])
    res = run_gpu(case, gkv, torch, cuda, out_dtype=torch.bfloat16 if p["bf16"] else None,
                  rotate_in_prefill=p["rot"])
    if p["rot"]:
        res["q"] = case.q_rot  # the append wrote no rotated Q
    check(case, res, rtol=RTOL + (2.0 ** -8 if p["bf16"] else 0.0))
