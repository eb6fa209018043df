"""Full-size decode layers on a gkv pool, for GPU tests at the benchmark configs' batch sizes.

The cache history is random bf16 written on the device (the host never holds
the whole cache). What the tests check:
- the append, over the whole batch and bit for bit: the pool arrays after the
  call equal a device copy of them taken before the call, with the new token's
  K and V (from the CPU oracle's kv_append of the same qkv rows) written at
  each sequence's slot, and nothing else changed;
- the attention of a sample of sequences against the CPU oracle, on their
  logical K/V gathered from the device cache through the block table.
"""
from __future__ import annotations

import numpy as np

from oracle import kv_oracle as O

D = 64
BT = 16


def device_copy(torch, gkv, ptr: int, n: int, dtype):
    """A torch copy of n elements of a pool array."""
    t = torch.empty(n, dtype=dtype, device="cuda")
    gkv.hip_memcpy_d2d(t.data_ptr(), ptr, n * t.element_size())
    return t


def host_table(torch, gkv, view, n_rows: int) -> np.ndarray:
    t = device_copy(torch, gkv, view.block_table, n_rows * view.table_stride, torch.int32)
    torch.cuda.synchronize()
    return t.view(n_rows, view.table_stride).cpu().numpy()


def bf16_bits_to_f32(torch, x):
    """int16 tensor of bf16 bits -> float32 (the bits as the high half)."""
    pair = torch.zeros(x.shape + (2,), dtype=torch.int16, device=x.device)
    pair[..., 1] = x
    return pair.view(torch.float32).squeeze(-1)


class PoolLayers:
    """A pool of n_layers (even layers = window W when W > 0) holding B
    sequences of context L[b] (seq_len L[b] + 1 after the append), random
    bf16 history N(0,1)*scale in every cache array, and per-layer qkv rows and
    sinks, all seeded."""

    def __init__(self, torch, gkv, L, n_layers=2, window=128, Hq=64, Hkv=8, scale=0.5,
                 seed=0):
        self.torch, self.gkv = torch, gkv
        self.L = np.asarray(L, np.int32)
        self.B = len(self.L)
        self.Hq, self.Hkv, self.scale = Hq, Hkv, scale
        self.seq_lens = self.L + 1
        self.max_len = int(self.seq_lens.max())
        need = int(((self.seq_lens + BT - 1) // BT).sum())
        self.pool = gkv.Pool(n_layers=n_layers, n_kv_heads=Hkv, max_seqs=self.B,
                             max_seq_len=self.max_len, window=window, num_blocks=need + 32,
                             shuffle_seed=seed + 1)
        for b in range(self.B):
            assert self.pool.seq_alloc() == b
            st = self.pool.reserve(b, int(self.seq_lens[b]))
            assert st == 0, gkv.status_string(st)
        self.pool.sync()
        dev = torch.device("cuda:0")
        self.views = [self.pool.view(li) for li in range(n_layers)]
        self.qkv, self.sinks = [], []
        for li, v in enumerate(self.views):
            n = v.num_blocks * Hkv * BT * D
            for j, base in enumerate((v.k, v.v)):
                g = torch.Generator(device=dev)
                g.manual_seed(seed * 1000 + 7 * li + j)
                t = torch.empty(n, dtype=torch.bfloat16, device=dev).normal_(0.0, scale,
                                                                             generator=g)
                gkv.hip_memcpy_d2d(base, t.data_ptr(), n * 2)
                torch.cuda.synchronize()
                del t
            rng = np.random.default_rng(seed * 100 + li)
            self.qkv.append((rng.standard_normal((self.B, (Hq + 2 * Hkv) * D)) * scale)
                            .astype(np.float32))
            self.sinks.append(rng.standard_normal(Hq).astype(np.float32))
        self.cos, self.sin = gkv.rope_table(self.max_len)
        t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(dev)  # noqa: E731
        self.cos_d, self.sin_d, self.lens_d = t(self.cos), t(self.sin), t(self.seq_lens)
        self.t = t

    def close(self):
        self.pool.close()

    def snapshot(self, li):
        """Device copies (int16 bits) of layer li's K and V arrays."""
        v = self.views[li]
        n = v.num_blocks * self.Hkv * BT * D
        k = device_copy(self.torch, self.gkv, v.k, n, self.torch.int16)
        vv = device_copy(self.torch, self.gkv, v.v, n, self.torch.int16)
        return k, vv

    def expected_after_append(self, li, k_before, v_before):
        """The pool arrays as the append must leave them: the before-copies with
        each sequence's new K (rotated) and V at its slot (CPU oracle bits)."""
        torch = self.torch
        v = self.views[li]
        _, _, kb, vb = O.kv_append(self.qkv[li], self.Hq, self.Hkv, self.cos, self.sin, self.L)
        table = host_table(torch, self.gkv, v, self.B)
        slot = self.L % v.ring if v.ring else self.L
        phys = table[np.arange(self.B), slot // BT].astype(np.int64)
        off = slot % BT
        koff = np.asarray(self.gkv.block_offsets("k"), np.int64)   # [16][64]
        voff = np.asarray(self.gkv.block_offsets("v"), np.int64)   # [64][16]
        g = np.arange(self.Hkv, dtype=np.int64)[None, :, None]
        head_base = (phys[:, None, None] * self.Hkv + g) * (BT * D)
        k_idx = head_base + koff[off][:, None, :]                   # [B, Hkv, 64]
        v_idx = head_base + voff[:, off].T[:, None, :]
        k_exp, v_exp = k_before.clone(), v_before.clone()
        k_exp[torch.from_numpy(k_idx.reshape(-1)).cuda()] = \
            torch.from_numpy(kb.reshape(-1).view(np.int16)).cuda()
        v_exp[torch.from_numpy(v_idx.reshape(-1)).cuda()] = \
            torch.from_numpy(vb.reshape(-1).view(np.int16)).cuda()
        return k_exp, v_exp

    def logical_kv(self, li, k_arr, v_arr, seqs):
        """fp32 [len(seqs), S, Hkv, 64] K and V of the listed sequences (slot
        order; S = the ring or the longest of them) from the int16 pool copies."""
        torch = self.torch
        v = self.views[li]
        table = host_table(torch, self.gkv, v, self.B)
        koff = torch.tensor(self.gkv.block_offsets("k"), device="cuda").reshape(-1)
        voff = torch.tensor(self.gkv.block_offsets("v"), device="cuda").reshape(-1)
        nb_all = v.num_blocks
        kk = k_arr.view(nb_all, self.Hkv, BT * D)
        vv = v_arr.view(nb_all, self.Hkv, BT * D)
        lens = self.seq_lens[seqs]
        S = v.ring if v.ring else int(lens.max())
        kc = np.zeros((len(seqs), S, self.Hkv, D), np.float32)
        vc = np.zeros((len(seqs), S, self.Hkv, D), np.float32)
        for i, b in enumerate(seqs):
            n = min(int(lens[i]), v.ring) if v.ring else int(lens[i])
            nb = (n + BT - 1) // BT
            blocks = torch.from_numpy(table[b, :nb].astype(np.int64)).cuda()
            kbl = kk[blocks][:, :, koff].view(nb, self.Hkv, BT, D)
            vbl = vv[blocks][:, :, voff].view(nb, self.Hkv, D, BT)
            kf, vf = bf16_bits_to_f32(torch, kbl), bf16_bits_to_f32(torch, vbl)
            kc[i, :n] = kf.permute(0, 2, 1, 3).reshape(nb * BT, self.Hkv, D)[:n].cpu().numpy()
            vc[i, :n] = vf.permute(0, 3, 1, 2).reshape(nb * BT, self.Hkv, D)[:n].cpu().numpy()
        return kc, vc

    def oracle_out(self, li, k_arr, v_arr, seqs):
        v = self.views[li]
        kc, vc = self.logical_kv(li, k_arr, v_arr, seqs)
        q_rot, _, _, _ = O.kv_append(self.qkv[li][seqs], self.Hq, self.Hkv, self.cos, self.sin,
                                     self.L[seqs])
        return O.decode_attention(q_rot, kc, vc, self.L[seqs], self.sinks[li], window=v.ring,
                                  ring=v.ring)
