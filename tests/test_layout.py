"""Block layouts of the pool, on the CPU: every layout is a permutation of a
head's block, the Python helpers agree with the test placement, and each
layout puts what one lane of the attention kernel needs in one 16-byte piece,
in lane order (the property the kernel's loads rely on)."""
import numpy as np

from kvcase import from_pool, k_block_offsets, to_pool, v_block_offsets, v_int8_offsets


def test_layouts_are_permutations(gkv):
    for kind in ("k", "v", "v_int8", "k_fp8"):
        off = np.array(gkv.block_offsets(kind)).reshape(-1)
        assert sorted(off.tolist()) == list(range(1024)), kind


def test_helpers_agree_with_test_placement(gkv):
    assert np.array_equal(np.array(gkv.block_offsets("k")), k_block_offsets())
    assert np.array_equal(np.array(gkv.block_offsets("v")), v_block_offsets())
    v8 = np.stack([v_int8_offsets(t) for t in range(16)], axis=1)   # [dim, token]
    assert np.array_equal(np.array(gkv.block_offsets("v_int8")), v8)


def test_k_lane_pieces(gkv):
    """Lane kg*16 + t, piece m (bytes m*1024 + lane*16): dims 32m+8kg..+7 of token t."""
    off = np.array(gkv.block_offsets("k"))        # [t][d] -> element
    for m in range(2):
        for lane in range(64):
            t, kg = lane % 16, lane // 16
            want = [off[t, 32 * m + 8 * kg + j] for j in range(8)]
            assert want == list(range(m * 512 + lane * 8, m * 512 + lane * 8 + 8))


def test_v_lane_pieces(gkv):
    """Lane kg*16 + i, half h: tokens 4kg..4kg+3 of dim i + 32h, then of dim i + 32h + 16."""
    off = np.array(gkv.block_offsets("v"))        # [d][t] -> element
    for h in range(2):
        for lane in range(64):
            i, kg = lane % 16, lane // 16
            want = [off[i + 32 * h + 16 * nn, 4 * kg + j] for nn in range(2) for j in range(4)]
            assert want == list(range(h * 512 + lane * 8, h * 512 + lane * 8 + 8))


def test_pool_round_trip():
    rng = np.random.default_rng(3)
    k = rng.integers(0, 65535, (5, 8, 16, 64)).astype(np.uint16)
    v = rng.integers(0, 65535, (5, 8, 64, 16)).astype(np.uint16)
    assert np.array_equal(from_pool(to_pool(k, "k"), "k"), k)
    assert np.array_equal(from_pool(to_pool(v, "v"), "v"), v)
    # one element lands where the offset table says
    pk = to_pool(k, "k")
    assert pk[2, 3, k_block_offsets()[7, 45]] == k[2, 3, 7, 45]


def test_k_fp8_lane_pieces(gkv):
    """e4m3 K: lane kg*16 + t reads bytes lane*16 .. +15: dims 8kg..+7 of token t
    (its first matrix-op piece), then dims 32+8kg..+7 (its second)."""
    off = np.array(gkv.block_offsets("k_fp8"))    # [t][d] -> byte
    for lane in range(64):
        t, kg = lane % 16, lane // 16
        want = [off[t, 8 * kg + j] for j in range(8)] + [off[t, 32 + 8 * kg + j] for j in range(8)]
        assert want == list(range(lane * 16, lane * 16 + 16))
