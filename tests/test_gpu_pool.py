"""The paged KV pool (gkv_pool_*): block accounting, all-or-nothing
reservation, reuse after free, window rings, device tables equal to the host
bookkeeping, and sizing from a byte budget."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def dev_table(torch, gkv, view, n_rows):
    t = torch.empty(n_rows * view.table_stride, dtype=torch.int32, device="cuda")
    gkv.hip_memcpy_d2d(t.data_ptr(), view.block_table, t.numel() * 4)
    torch.cuda.synchronize()
    return t.view(n_rows, view.table_stride).cpu().numpy()


def test_block_accounting_and_tables(gkv, cuda):
    import torch
    pool = gkv.Pool(n_layers=2, n_kv_heads=8, max_seqs=4, max_seq_len=100, window=32,
                    num_blocks=12, shuffle_seed=5)
    try:
        assert pool.num_blocks() == 12 and pool.free_blocks() == 12
        s = [pool.seq_alloc() for _ in range(3)]
        assert sorted(s) == [0, 1, 2]
        assert pool.reserve(s[0], 33) == 0          # 3 blocks
        assert pool.reserve(s[1], 16) == 0          # 1 block
        assert pool.reserve(s[1], 10) == 0          # never shrinks
        assert pool.free_blocks() == 8
        b0, b1 = pool.seq_blocks(s[0]), pool.seq_blocks(s[1])
        assert len(b0) == 3 and len(b1) == 1
        assert len(set(b0) | set(b1)) == 4 and all(0 <= x < 12 for x in list(b0) + list(b1))
        # all or nothing: 9 more blocks do not fit, nothing is taken
        assert pool.reserve(s[2], 9 * 16) == gkv.GKV_ERR_CAPACITY
        assert pool.free_blocks() == 8 and len(pool.seq_blocks(s[2])) == 0
        # beyond the table row (max_seq_len 100 -> 7 blocks)
        assert pool.reserve(s[2], 101 + 16) == gkv.GKV_ERR_CAPACITY
        pool.sync()
        full = pool.view(1)
        assert full.ring == 0 and full.num_blocks == 12
        t = dev_table(torch, gkv, full, 4)
        assert list(t[s[0], :3]) == list(b0) and (t[s[0], 3:] == -1).all()
        assert list(t[s[1], :1]) == list(b1)
        assert (t[s[2]] == -1).all()
        ring = pool.view(0)
        assert ring.ring == 32 and ring.table_stride == 2 and ring.num_blocks == 8
        rt = dev_table(torch, gkv, ring, 4)
        assert sorted(rt.reshape(-1).tolist()) == list(range(8))  # fixed ring per sequence id
        # free returns the blocks, and they are handed out again
        assert pool.free(s[0]) == 0
        assert pool.free_blocks() == 11
        assert pool.free(s[0]) == gkv.GKV_ERR_BLOCK     # not live any more
        s3 = pool.seq_alloc()
        assert pool.reserve(s3, 7 * 16) == 0      # a full table row (7 blocks)
        assert pool.reserve(s[2], 4 * 16) == 0
        assert pool.free_blocks() == 0
        pool.sync()
        t = dev_table(torch, gkv, pool.view(1), 4)
        used = [x for x in t.reshape(-1).tolist() if x >= 0]
        assert sorted(used) == list(range(12))
        # a view starting at a later sequence id shifts the table rows
        v2 = pool.view(1, first_seq=2)
        assert v2.block_table == full.block_table + 2 * full.table_stride * 4
    finally:
        pool.close()


def test_incremental_sync_tracks_the_host_tables(gkv, cuda):
    """gkv_pool_sync sends only the changed entries, asynchronously: after
    rounds of random reserves and frees (a free and a new reserve of the same
    entries within one sync among them, and more changes than the staging
    buffer first holds), the device table equals the host bookkeeping."""
    import torch
    rng = np.random.default_rng(7)
    S, L = 64, 2000
    per = (L + 15) // 16
    pool = gkv.Pool(n_layers=1, n_kv_heads=8, max_seqs=S, max_seq_len=L, window=0,
                    num_blocks=S * per, shuffle_seed=9)
    try:
        live = set()
        stream = torch.cuda.Stream()
        for rnd in range(12):
            for _ in range(40):
                if live and rng.random() < 0.3:
                    s = int(rng.choice(sorted(live)))
                    assert pool.free(s) == 0
                    live.discard(s)
                elif len(live) < S:
                    s = pool.seq_alloc()
                    live.add(s)
                    assert pool.reserve(s, int(rng.integers(1, L + 1))) == 0
            for s in list(live)[:5]:  # grow some
                assert pool.reserve(s, L) == 0
            pool.sync(stream)
            stream.synchronize()
            t = dev_table(torch, gkv, pool.view(0), S)
            for s in range(S):
                want = list(pool.seq_blocks(s)) if s in live else []
                assert list(t[s, :len(want)]) == want, f"round {rnd} seq {s}"
                assert (t[s, len(want):] == -1).all(), f"round {rnd} seq {s}"
    finally:
        pool.close()


def test_sequence_ids_and_errors(gkv, cuda):
    pool = gkv.Pool(n_layers=1, n_kv_heads=8, max_seqs=2, max_seq_len=64, window=0,
                    num_blocks=8)
    try:
        a, b = pool.seq_alloc(), pool.seq_alloc()
        with pytest.raises(RuntimeError):
            pool.seq_alloc()                      # only 2 sequence ids
        assert pool.reserve(5, 10) == gkv.GKV_ERR_BLOCK
        assert pool.reserve(a, -1) == gkv.GKV_ERR_ARG
        assert pool.free(a) == 0
        assert pool.seq_alloc() == a              # the id comes back
        assert pool.reserve(b, 64) == 0 and pool.free_blocks() == 4
    finally:
        pool.close()


def test_budget_sizing(gkv, cuda):
    # layers 0 and 2 are window layers, layer 1 full: 8 heads x 2 KB x 2 (K, V)
    # = 32 KB per block and layer; the rings take 2 layers x 4 seqs x 2 blocks
    # x 32 KB, the tables (4 x 16 + 4 x 2) x 4 B
    budget = 100 * 32768 + 2 * 4 * 2 * 32768 + 4096
    pool = gkv.Pool(n_layers=3, n_kv_heads=8, max_seqs=4, max_seq_len=256, window=32,
                    bytes_budget=budget)
    try:
        nb = pool.num_blocks()
        assert nb == 100
        assert pool.device_bytes() <= budget
    finally:
        pool.close()
