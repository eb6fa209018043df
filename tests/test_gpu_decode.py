"""GPU parity of the KV append and the decode attention against the CPU oracle.

Appends are compared bit for bit (every byte of the paged cache, including the
NaN-poisoned slots that must stay untouched); attention outputs within
max-abs 2e-3 + rel 1e-2 (bf16 cache, fp32 accumulate), the tolerance of the
north-star contract. Inputs are seeded; shapes follow the benchmark configs
(reduced batch where the CPU oracle has to run the whole batch).
"""
import numpy as np
import pytest

from kvcase import DecodeCase, allclose_report, from_pool

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def run_gpu(case: DecodeCase, gkv, torch, device, split_tokens=0, out_dtype=None,
            rotate_in_attention=True, product_table=True, layer_call=False):
    cos = sin = None
    if product_table:
        cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, device, cos, sin)
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring,
                          v_scale=dev["vs"])
    q_out = None
    if not rotate_in_attention:
        q_out = torch.empty(case.B, case.Hq * 64, dtype=torch.float32, device=device)
    if not layer_call:
        gkv.kv_append(dev["qkv"], case.Hq, dev["cos"], dev["sin"], dev["pos"], view,
                      seq_lens=dev["seq_lens"], q_out=q_out, dev_err=dev["err"])
    max_len = int(case.seq_lens.max())
    ws_bytes = gkv.workspace_bytes(case.B, case.Hkv, max_len, case.window, split_tokens)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=device)
    out = torch.full((case.B, case.Hq * 64), float("nan"),
                     dtype=out_dtype or torch.float32, device=device)
    if layer_call:
        gkv.decode_layer(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                         dev["cos"], dev["sin"], window=case.window, split_tokens=split_tokens,
                         workspace=ws, dev_err=dev["err"])
    elif rotate_in_attention:
        gkv.decode_attention(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                             window=case.window, cos_tab=dev["cos"], sin_tab=dev["sin"],
                             split_tokens=split_tokens, workspace=ws, dev_err=dev["err"])
    else:
        gkv.decode_attention(q_out, dev["seq_lens"], max_len, view, dev["sinks"], out,
                             window=case.window, split_tokens=split_tokens, workspace=ws,
                             dev_err=dev["err"])
    torch.cuda.synchronize()
    res = {
        "k": from_pool(dev["k"].cpu().numpy().view(np.uint16), "k"),
        "v": dev["v"].cpu().numpy() if case.v_int8 else
        from_pool(dev["v"].cpu().numpy().view(np.uint16), "v"),
        "vs": dev["vs"].cpu().numpy() if case.v_int8 else None,
        "out": out.float().cpu().numpy().reshape(case.B, case.Hq, 64),
        "err": int(dev["err"].cpu().item()),
    }
    if q_out is not None:
        res["q_rot"] = q_out.cpu().numpy().reshape(case.B, case.Hq, 64)
    return res


def check_case(case, res, atol=ATOL, rtol=RTOL):
    assert res["err"] == 0
    assert np.array_equal(res["k"], case.k_expect), "K cache bytes differ"
    assert np.array_equal(res["v"], case.v_expect), "V cache bytes differ"
    if case.v_int8:
        assert np.array_equal(res["vs"].view(np.uint32), case.vs_expect.view(np.uint32)), \
            "V scales differ"
    ref = case.oracle_out()
    assert np.isfinite(res["out"]).all()
    bad, worst = allclose_report(res["out"], ref, atol, rtol)
    assert bad == 0, f"{bad} outputs out of tolerance, max abs err {worst:.3e}"
    return worst


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def lens_uniform(rng, B, lo, hi):
    return rng.integers(lo, hi + 1, size=B).astype(np.int32)


# ---- config 1: B=4, H_q=8, H_kv=2, lengths U[1,256] ----------------------------

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_config1_tiny_gqa(gkv, cuda, torch_mod, seed):
    rng = np.random.default_rng(100 + seed)
    L = lens_uniform(rng, 4, 0, 255)  # 1..256 tokens after the append
    case = DecodeCase(4, 8, 2, L, window=0, seed=seed)
    print(f"config1 seed={seed} L={L.tolist()}", flush=True)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))


@pytest.mark.parametrize("window", [0, 128])
def test_config1_window_layer(gkv, cuda, torch_mod, window):
    rng = np.random.default_rng(7)
    L = np.array([0, 127, 128, 255], np.int32)
    case = DecodeCase(4, 8, 2, L, window=window, seed=3)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))


# ---- config 2 / 3 shapes at reduced batch --------------------------------------

def test_config2_full_layer_reduced_batch(gkv, cuda, torch_mod):
    rng = np.random.default_rng(2)
    B = 48
    L = lens_uniform(rng, B, 128, 2048)
    case = DecodeCase(B, 64, 8, L, window=0, scale=0.5, seed=22)
    print(f"config2 B={B}", flush=True)
    worst = check_case(case, run_gpu(case, gkv, torch_mod, cuda))
    print(f"max abs err {worst:.2e}")


def test_config3_window_layer_reduced_batch(gkv, cuda, torch_mod):
    rng = np.random.default_rng(3)
    B = 64
    L = lens_uniform(rng, B, 0, 4095)
    L[:4] = [0, 126, 127, 128]  # partial, exactly full, and wrapped rings
    case = DecodeCase(B, 64, 8, L, window=128, scale=0.5, seed=33)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))


@pytest.mark.parametrize("window", [0, 128])
def test_decode_layer_call_matches_two_calls(gkv, cuda, torch_mod, window):
    """gkv_decode_layer (append fused into the prepare launch) writes the same
    cache bytes as gkv_kv_append and the same output bits as
    gkv_decode_attention, and both match the oracle."""
    rng = np.random.default_rng(60 + window)
    B = 40
    L = lens_uniform(rng, B, 0, 3000)
    L[:3] = [0, 127, 128]
    case = DecodeCase(B, 64, 8, L, window=window, scale=0.5, seed=61 + window)
    fused = run_gpu(case, gkv, torch_mod, cuda, layer_call=True)
    check_case(case, fused)
    two = run_gpu(case, gkv, torch_mod, cuda)
    assert np.array_equal(fused["out"].view(np.uint32), two["out"].view(np.uint32))


# ---- int8 V (the reference's quantized-V cache) ---------------------------------

@pytest.mark.parametrize("window", [0, 128])
def test_int8_v_cache(gkv, cuda, torch_mod, window):
    """Append bit-exact (codes and scales of the reference's rule) and
    attention within tolerance of the oracle on the dequantized values."""
    rng = np.random.default_rng(70 + window)
    B = 40
    L = lens_uniform(rng, B, 0, 2100)
    L[:4] = [0, 15, 127, 128]
    case = DecodeCase(B, 64, 8, L, window=window, scale=0.5, seed=71 + window, v_int8=True)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))
    check_case(case, run_gpu(case, gkv, torch_mod, cuda, layer_call=True))


def test_int8_v_config1_and_split_sizes(gkv, cuda, torch_mod):
    L = np.array([1, 77, 200, 256], np.int32)
    case = DecodeCase(4, 8, 2, L, window=0, scale=1.0, seed=72, v_int8=True)
    for split in (0, 32, 128):
        check_case(case, run_gpu(case, gkv, torch_mod, cuda, split_tokens=split))


# ---- edges ---------------------------------------------------------------------

EDGE_LENS = [0, 1, 14, 15, 16, 17, 31, 32, 33, 127, 128, 129, 511, 512, 513, 1023, 1024, 1535]


def test_edge_lengths(gkv, cuda, torch_mod):
    L = np.array(EDGE_LENS, np.int32)
    case = DecodeCase(len(L), 64, 8, L, window=0, scale=0.5, seed=44)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))


@pytest.mark.parametrize("split_tokens", [0, 16384])
def test_long_sequences(gkv, cuda, torch_mod, split_tokens):
    """Contexts far past one range: 40k and 20k tokens beside short ones. With
    the balanced split a 40k context spans over a hundred ranges, all merged
    by the combine; with 16384-token ranges (the largest a range holds) the
    ranges' block ids and step records fill their LDS slabs."""
    L = np.array([40000, 5, 20000, 16391], np.int32)
    case = DecodeCase(len(L), 64, 8, L, window=0, scale=0.5, seed=57)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda, split_tokens=split_tokens))


@pytest.mark.parametrize("window", [0, 32])
def test_largest_batch(gkv, cuda, torch_mod, window):
    """8192 sequences, the most one call takes (the split's prefix sums and
    lengths sit in LDS), short contexts, through gkv_decode_layer."""
    rng = np.random.default_rng(58 + window)
    L = lens_uniform(rng, 8192, 0, 48)
    case = DecodeCase(len(L), 64, 8, L, window=window, scale=0.5, seed=59)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda, layer_call=True))


@pytest.mark.parametrize("split_tokens", [128, 256, 512, 1024])
def test_split_sizes_agree(gkv, cuda, torch_mod, split_tokens):
    L = np.array([5, 300, 700, 1300, 2047], np.int32)
    case = DecodeCase(len(L), 64, 8, L, window=0, scale=0.5, seed=55)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda, split_tokens=split_tokens))


def test_rotated_q_path_and_bf16_output(gkv, cuda, torch_mod):
    L = np.array([3, 200, 900, 64], np.int32)
    case = DecodeCase(len(L), 64, 8, L, window=0, scale=0.5, seed=66)
    res = run_gpu(case, gkv, torch_mod, cuda, rotate_in_attention=False)
    assert np.array_equal(res["q_rot"].view(np.uint32), case.q_rot.view(np.uint32))
    check_case(case, res)
    res16 = run_gpu(case, gkv, torch_mod, cuda, out_dtype=torch_mod.bfloat16)
    check_case(case, res16)


def test_large_scores_and_sinks(gkv, cuda, torch_mod):
    """Peaky softmax: large q/k (scores up to ~±100) and large sinks."""
    L = np.array([50, 400, 1100], np.int32)
    case = DecodeCase(len(L), 64, 8, L, window=0, scale=2.5, seed=77, sink_scale=8.0)
    check_case(case, run_gpu(case, gkv, torch_mod, cuda))


def test_physical_placement_does_not_matter(gkv, cuda, torch_mod):
    """Same logical cache under two different block permutations: outputs
    identical bit for bit."""
    L = np.array([40, 700, 1500], np.int32)
    a = DecodeCase(3, 64, 8, L, window=0, scale=0.5, seed=88, extra_blocks=3)
    b = DecodeCase(3, 64, 8, L, window=0, scale=0.5, seed=88, extra_blocks=3)
    # re-place b's blocks with another permutation
    perm = np.random.default_rng(1).permutation(b.num_blocks).astype(np.int32)
    inv_k = np.empty_like(b.k)
    inv_v = np.empty_like(b.v)
    inv_k[perm] = b.k
    inv_v[perm] = b.v
    b.k, b.v = inv_k, inv_v
    b.table = np.where(b.table >= 0, perm[np.maximum(b.table, 0)], -1).astype(np.int32)
    ek, ev = np.empty_like(b.k_expect), np.empty_like(b.v_expect)
    ek[perm] = b.k_expect
    ev[perm] = b.v_expect
    b.k_expect, b.v_expect = ek, ev
    ra = run_gpu(a, gkv, torch_mod, cuda)
    rb = run_gpu(b, gkv, torch_mod, cuda)
    check_case(b, rb)
    assert np.array_equal(ra["out"].view(np.uint32), rb["out"].view(np.uint32))


def test_bad_block_id_is_flagged_not_faulted(gkv, cuda, torch_mod):
    L = np.array([100, 100], np.int32)
    case = DecodeCase(2, 64, 8, L, window=0, scale=0.5, seed=99)
    case.table[1, 2] = case.num_blocks + 5  # out of range (a history block)
    res = run_gpu(case, gkv, torch_mod, cuda)
    assert res["err"] & gkv.DEVERR_BLOCK_ID
    # sequence 0 is unaffected
    ref = case.oracle_out()
    bad, _ = allclose_report(res["out"][0], ref[0])
    assert bad == 0
    assert np.isfinite(res["out"]).all()


def test_repeated_split_launches_reuse_the_plan(gkv, cuda, torch_mod):
    """One prepare, then split + combine three times over the same workspace:
    every repeat gives the same bits, within tolerance of the oracle."""
    rng = np.random.default_rng(87)
    L = lens_uniform(rng, 48, 100, 2000)
    case = DecodeCase(48, 64, 8, L, window=0, scale=0.5, seed=88)
    torch = torch_mod
    dev = case.to_device(torch, cuda, *gkv.rope_table(case.cos.shape[0]))
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv)
    gkv.kv_append(dev["qkv"], case.Hq, dev["cos"], dev["sin"], dev["pos"], view,
                  seq_lens=dev["seq_lens"], dev_err=dev["err"])
    max_len = int(case.seq_lens.max())
    ws = torch.empty(gkv.workspace_bytes(case.B, case.Hkv, max_len), dtype=torch.uint8,
                     device=cuda)
    kw = dict(cos_tab=dev["cos"], sin_tab=dev["sin"], workspace=ws, dev_err=dev["err"])
    outs = []
    for i in range(3):
        out = torch.full((case.B, case.Hq * 64), float("nan"), dtype=torch.float32, device=cuda)
        stages = ("prepare", "split", "combine") if i == 0 else ("split", "combine")
        for st in stages:
            gkv.decode_attention(dev["qkv"], dev["seq_lens"], max_len, view, dev["sinks"], out,
                                 stage=st, **kw)
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy().reshape(case.B, case.Hq, 64))
    assert int(dev["err"].item()) == 0
    bad, worst = allclose_report(outs[0], case.oracle_out(), ATOL, RTOL)
    assert bad == 0, f"{bad} outputs out of tolerance (max err {worst:.3e})"
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


# ---- window layers: ranges of whole sequences, no combine -------------------------

def test_window_layer_whole_sequence_ranges(gkv, cuda, torch_mod):
    """A window layer with the balanced split cuts the stream only between
    sequences (more sequences than workgroups here, lengths from 1 token to
    past the ring), launches no combine, and matches the oracle. Each sequence
    is then computed by one wave in a fixed order whatever the partition: with
    some sequences emptied (length 0, output 0) the others keep their bits.
    The staged launches on the same layer still run the combine and agree
    within tolerance."""
    torch = torch_mod
    rng = np.random.default_rng(90)
    B = 600
    L = lens_uniform(rng, B, 0, 300)
    L[:6] = [0, 1, 30, 126, 127, 128]
    case = DecodeCase(B, 64, 8, L, window=128, scale=0.5, seed=91)
    max_len = int(case.seq_lens.max())
    assert not gkv.layer_combines(B, 8, max_len, 128, 0)
    assert gkv.layer_combines(B, 8, max_len, 0, 0)
    assert gkv.layer_combines(B, 8, max_len, 128, 256)
    res = run_gpu(case, gkv, torch, cuda, layer_call=True)
    check_case(case, res)

    # the cache now holds every sequence's new token: attention only, first
    # with the same lengths, then with some of them set to 0
    cos, sin = gkv.rope_table(case.cos.shape[0])
    dev = case.to_device(torch, cuda, cos, sin)
    view = gkv.cache_view(dev["k"], dev["v"], dev["table"], case.Hkv, ring=case.ring)
    gkv.kv_append(dev["qkv"], case.Hq, dev["cos"], dev["sin"], dev["pos"], view,
                  seq_lens=dev["seq_lens"], dev_err=dev["err"])
    ws = torch.empty(gkv.workspace_bytes(B, 8, max_len, 128, 0), dtype=torch.uint8, device=cuda)

    def attend(lens, stages=("both",)):
        out = torch.full((B, case.Hq * 64), float("nan"), dtype=torch.float32, device=cuda)
        lens_d = torch.from_numpy(lens.astype(np.int32)).to(cuda)
        for st in stages:
            gkv.decode_attention(dev["qkv"], lens_d, max_len, view, dev["sinks"], out,
                                 window=128, cos_tab=dev["cos"], sin_tab=dev["sin"],
                                 workspace=ws, dev_err=dev["err"], stage=st)
        torch.cuda.synchronize()
        return out.cpu().numpy().reshape(B, case.Hq, 64)

    full = attend(case.seq_lens)
    assert np.array_equal(full.view(np.uint32), res["out"].view(np.uint32))
    lens0 = case.seq_lens.copy()
    empty = rng.choice(B, 50, replace=False)
    lens0[empty] = 0
    part = attend(lens0)
    keep = np.setdiff1d(np.arange(B), empty)
    assert np.array_equal(part[empty], np.zeros_like(part[empty]))
    assert np.array_equal(part[keep].view(np.uint32), full[keep].view(np.uint32))
    staged = attend(case.seq_lens, ("prepare", "split", "combine"))
    bad, worst = allclose_report(staged, case.oracle_out())
    assert bad == 0, f"staged: {bad} outputs out of tolerance ({worst:.3e})"
    assert int(dev["err"].cpu().item()) == 0
