"""GPU parity of the exact path (gkv_rope_exact, gkv_kv_write_exact,
gkv_attention_exact) over fp32 caches: bit for bit against the CPU oracle
(oracle/kv_oracle.c, itself bit-exact with run.cpp's forward), and, where the
reference's own run.cpp is built (oracle/_ref), against its forward() on whole
decode steps. Every comparison is of the fp32 bit patterns."""
import numpy as np
import pytest

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

D = 64


def bits(x):
    return np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)


def assert_bits_equal(got, want, what):
    g, w = bits(got), bits(want)
    bad = np.nonzero(g != w)
    assert g.shape == w.shape, what
    assert bad[0].size == 0, (f"{what}: {bad[0].size} of {g.size} values differ, first at "
                              f"{tuple(int(i[0]) for i in bad)}: "
                              f"{got[tuple(i[0] for i in bad)]} vs {want[tuple(i[0] for i in bad)]}")


def test_rope_exact_bit_exact(gkv, cuda):
    import torch
    rng = np.random.default_rng(11)
    B, Hq, Hkv = 64, 64, 8
    qkv = (rng.standard_normal((B, (Hq + 2 * Hkv) * D)) * 0.5).astype(np.float32)
    pos = rng.integers(0, 4096, size=B).astype(np.int32)
    cos, sin = gkv.rope_table(4096)
    print(f"rope_exact B={B} heads={Hq + Hkv}", flush=True)
    d_qkv = torch.from_numpy(qkv).to(cuda)
    d_cos, d_sin = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    gkv.rope_exact(d_qkv, d_cos, d_sin, Hq + Hkv, positions=torch.from_numpy(pos).to(cuda))
    # one position for every row, the tables' row passed as the reference does
    d_one = torch.from_numpy(qkv).to(cuda)
    gkv.rope_exact(d_one, d_cos[1234], d_sin[1234], Hq + Hkv)
    torch.cuda.synchronize()
    got, got_one = d_qkv.cpu().numpy(), d_one.cpu().numpy()
    n_rot = (Hq + Hkv) * D
    for b in range(B):
        want = O.rotate(qkv[b, :n_rot], cos[pos[b]], sin[pos[b]])
        assert_bits_equal(got[b, :n_rot], want, f"row {b}")
        assert_bits_equal(got_one[b, :n_rot], O.rotate(qkv[b, :n_rot], cos[1234], sin[1234]),
                          f"row {b}, pos 1234")
    assert_bits_equal(got[:, n_rot:], qkv[:, n_rot:], "V untouched")


def test_kv_write_exact(gkv, cuda):
    import torch
    rng = np.random.default_rng(12)
    B, Hq, Hkv, slots, W = 16, 64, 8, 128, 128
    kv_dim = Hkv * D
    row = (Hq + 2 * Hkv) * D
    qkv = rng.standard_normal((B, row)).astype(np.float32)
    pos = rng.integers(0, 4096, size=B).astype(np.int32)
    pos[3] = -1  # no slot: skipped and flagged
    print("kv_write_exact ring", flush=True)
    d_qkv = torch.from_numpy(qkv).to(cuda)
    kc = torch.full((B, slots, kv_dim), float("nan"), device=cuda)
    vc = torch.full((B, slots, kv_dim), float("nan"), device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    gkv.kv_write_exact(d_qkv, Hq * D, Hq * D + kv_dim, kc, vc, kv_dim,
                       positions=torch.from_numpy(pos).to(cuda), window=W, dev_err=err)
    # one slot for every row
    kc2 = torch.full((B, 40, kv_dim), float("nan"), device=cuda)
    vc2 = torch.full((B, 40, kv_dim), float("nan"), device=cuda)
    gkv.kv_write_exact(d_qkv, Hq * D, Hq * D + kv_dim, kc2, vc2, kv_dim, slot=37)
    torch.cuda.synchronize()
    k, v, k2, v2 = (t.cpu().numpy() for t in (kc, vc, kc2, vc2))
    assert int(err.item()) == gkv.DEVERR_LENGTH
    for b in range(B):
        written = np.zeros(slots, bool)
        if pos[b] >= 0:
            s = pos[b] % W
            written[s] = True
            assert_bits_equal(k[b, s], qkv[b, Hq * D:Hq * D + kv_dim], f"K row {b}")
            assert_bits_equal(v[b, s], qkv[b, Hq * D + kv_dim:], f"V row {b}")
        assert np.isnan(k[b, ~written]).all() and np.isnan(v[b, ~written]).all(), b
        assert_bits_equal(k2[b, 37], qkv[b, Hq * D:Hq * D + kv_dim], f"K row {b} slot 37")
        assert_bits_equal(v2[b, 37], qkv[b, Hq * D + kv_dim:], f"V row {b} slot 37")
        assert np.isnan(np.delete(k2[b], 37, axis=0)).all()


def _attention_case(seed, B, Hq, Hkv, lens_lo, lens_hi, window=0, slots=None):
    rng = np.random.default_rng(seed)
    pos = rng.integers(lens_lo, lens_hi + 1, size=B).astype(np.int32) - 1
    if slots is None:
        slots = window if window > 0 else int(pos.max()) + 1 + 5
    q = (rng.standard_normal((B, Hq, D)) * 0.5).astype(np.float32)
    kc = np.full((B, slots, Hkv, D), np.nan, np.float32)
    vc = np.full((B, slots, Hkv, D), np.nan, np.float32)
    for b in range(B):
        p = pos[b]
        t0 = max(0, p - window + 1) if window > 0 else 0
        for t in range(t0, p + 1):
            s = t % window if window > 0 else t
            kc[b, s] = rng.standard_normal((Hkv, D)) * 0.5
            vc[b, s] = rng.standard_normal((Hkv, D)) * 0.5
    sinks = rng.standard_normal(Hq).astype(np.float32)
    return pos, q, kc, vc, sinks, slots


@pytest.mark.parametrize("name,B,Hq,Hkv,lo,hi,window", [
    ("config1", 4, 8, 2, 1, 256, 0),           # the CPU-runnable case: B=4, Hq=8, Hkv=2
    ("config2_shape", 6, 64, 8, 128, 2048, 0),   # gpt-oss-20b shape, fewer sequences
    ("window_ring", 8, 64, 8, 1, 4096, 128),     # 128-slot rings, partial and full windows
    ("long", 2, 16, 2, 9000, 12000, 0),          # score rows past a workgroup's LDS for 8 heads
    ("group16", 3, 32, 2, 1, 3000, 0),           # 16 query heads per kv head (1024 threads)
    ("group1", 3, 4, 4, 1, 700, 64),             # one query head per kv head, a 64-slot ring
])
def test_attention_exact_bit_exact(gkv, cuda, name, B, Hq, Hkv, lo, hi, window):
    import torch
    pos, q, kc, vc, sinks, slots = _attention_case(sum(map(ord, name)), B, Hq, Hkv, lo, hi, window)
    print(f"attention_exact {name}: B={B} Hq={Hq} Hkv={Hkv} slots={slots} window={window} "
          f"max pos {pos.max()}", flush=True)
    want = O.decode_attention(q, kc, vc, pos, sinks, window=window, ring=window)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    out = torch.full((B, Hq * D), float("nan"), device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    gkv.attention_exact(d(q.reshape(B, Hq * D)), Hq, Hkv, d(kc.reshape(B, slots, Hkv * D)),
                        d(vc.reshape(B, slots, Hkv * D)), d(sinks), out, positions=d(pos),
                        max_pos=int(pos.max()), window=window, dev_err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    assert_bits_equal(out.cpu().numpy().reshape(B, Hq, D), want, name)


def test_attention_exact_one_position_and_flags(gkv, cuda):
    """One position for every row (the reference engine's call), and a row
    past the host bound: zeros and the length flag, the others unchanged."""
    import torch
    B, Hq, Hkv = 4, 64, 8
    pos, q, kc, vc, sinks, slots = _attention_case(5, B, Hq, Hkv, 300, 300, 0, slots=512)
    print("attention_exact one position", flush=True)
    want = O.decode_attention(q, kc, vc, pos, sinks)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    dq, dk, dv = (d(q.reshape(B, -1)), d(kc.reshape(B, slots, -1)), d(vc.reshape(B, slots, -1)))
    out = torch.full((B, Hq * D), float("nan"), device=cuda)
    gkv.attention_exact(dq, Hq, Hkv, dk, dv, d(sinks), out, pos=299)
    p2 = pos.copy()
    p2[2] = 600  # beyond max_pos (and the cache): zeros and GKV_DEVERR_LENGTH
    out2 = torch.full((B, Hq * D), float("nan"), device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    gkv.attention_exact(dq, Hq, Hkv, dk, dv, d(sinks), out2, positions=d(p2), max_pos=299,
                        dev_err=err)
    torch.cuda.synchronize()
    assert_bits_equal(out.cpu().numpy().reshape(B, Hq, D), want, "pos 299")
    o2 = out2.cpu().numpy().reshape(B, Hq, D)
    assert int(err.item()) == gkv.DEVERR_LENGTH
    assert (o2[2] == 0).all()
    keep = [0, 1, 3]
    assert_bits_equal(o2[keep], want[keep], "other rows")


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref (the reference's run.cpp) not built")
@pytest.mark.parametrize("window_layer", [False, True])
def test_exact_step_matches_reference_forward(gkv, cuda, window_layer):
    """rope_exact + kv_write_exact + attention_exact on decode rows, bit for
    bit with the reference's own run.cpp forward() (compiled from its sources
    in oracle/_ref): the rotated key in the cache and the attention output."""
    import torch
    rng = np.random.default_rng(21 + window_layer)
    Hq, Hkv, W = 64, 8, 128
    kv_dim = Hkv * D
    row = (Hq + 2 * Hkv) * D
    pos = np.array([0, 1, 127, 128, 129, 700, 1500, 2047], np.int32)
    B = len(pos)
    slots = W if window_layer else 2048
    window = W if window_layer else 0
    qkv = (rng.standard_normal((B, row)) * 0.5).astype(np.float32)
    sinks = rng.standard_normal(Hq).astype(np.float32)
    k_hist = [(rng.standard_normal((p, kv_dim)) * 0.5).astype(np.float32) for p in pos]
    v_hist = [(rng.standard_normal((p, kv_dim)) * 0.5).astype(np.float32) for p in pos]
    kc = np.full((B, slots, kv_dim), np.nan, np.float32)
    vc = np.full((B, slots, kv_dim), np.nan, np.float32)
    for b, p in enumerate(pos):
        for t in range(max(0, p - W + 1) if window_layer else 0, p):
            s = t % W if window_layer else t
            kc[b, s], vc[b, s] = k_hist[b][t], v_hist[b][t]
    print(f"exact step vs run.cpp window_layer={window_layer}", flush=True)
    cos, sin = gkv.rope_table(2048)
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(cuda)
    d_qkv, d_kc, d_vc, d_pos = d(qkv), d(kc), d(vc), d(pos)
    out = torch.full((B, Hq * D), float("nan"), device=cuda)
    err = torch.zeros(1, dtype=torch.int32, device=cuda)
    gkv.rope_exact(d_qkv, d(cos), d(sin), Hq + Hkv, positions=d_pos)
    gkv.kv_write_exact(d_qkv, Hq * D, Hq * D + kv_dim, d_kc, d_vc, kv_dim, positions=d_pos,
                       window=window, dev_err=err)
    gkv.attention_exact(d_qkv, Hq, Hkv, d_kc, d_vc, d(sinks), out, positions=d_pos,
                        max_pos=int(pos.max()), window=window, dev_err=err)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got_out = out.cpu().numpy().reshape(B, Hq, D)
    got_k = d_kc.cpu().numpy()
    for b, p in enumerate(pos):
        want_out, want_k = O.ref_decode_one(qkv[b], k_hist[b], v_hist[b], sinks, int(p), Hq, Hkv,
                                            window=W, window_layer=window_layer)
        s = p % W if window_layer else p
        assert_bits_equal(got_k[b, s].reshape(Hkv, D), want_k, f"cached key, pos {p}")
        assert_bits_equal(got_out[b], want_out, f"output, pos {p}")
