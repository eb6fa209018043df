"""The CPU oracle against the reference's golden vectors, the reference build
(when oracle/_ref is present) and the closed forms of the mathematics."""
import hashlib

import numpy as np
import pytest

from oracle import kv_oracle as O


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ---- RoPE angles (run.cpp:422-504) ------------------------------------------

def test_rope_table_matches_golden(golden):
    c, s = O.rope_table(4097)
    pos = golden["table_positions"]
    assert np.array_equal(bits(c[pos]), bits(golden["table_cos"]))
    assert np.array_equal(bits(s[pos]), bits(golden["table_sin"]))
    digest = hashlib.sha256(c.tobytes() + s.tobytes()).hexdigest()
    assert digest == bytes(golden["table_sha256"]).decode()


def test_rope_closed_forms():
    conc, inv = O.yarn()
    assert conc == np.float32(np.float32(0.1) * np.float32(np.log(32.0)) + np.float32(1.0))
    assert abs(conc - (0.1 * np.log(32) + 1)) < 1e-6
    assert inv[0] == 1.0                      # extrapolation region: 1 / base^0
    assert np.all(np.diff(inv) < 0)           # strictly decreasing frequencies
    c, s = O.rope_table(2)
    assert np.all(c[0] == np.float32(conc)) and np.all(s[0] == 0)
    # interpolation region: inv_freq = 1 / (32 * base^(2i/64)) for the last index
    i = 31
    assert abs(inv[i] - 1.0 / (32 * 150000.0 ** (2 * i / 64))) < 1e-6 * inv[i]


def test_rotate_matches_golden(golden):
    c, s = O.rope_table(4097)
    for i, p in enumerate(golden["rot_pos"]):
        got = O.rotate(golden["rot_in"][i].reshape(-1), c[p], s[p]).reshape(4, 64)
        assert np.array_equal(bits(got), bits(golden["rot_out"][i]))


def test_rotate_is_scaled_rotation():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(64 * 3).astype(np.float32)
    c, s = O.rope_table(500)
    conc, _ = O.yarn()
    y = O.rotate(x, c[499], s[499]).reshape(3, 2, 32).astype(np.float64)
    x3 = x.reshape(3, 2, 32).astype(np.float64)
    n_in = x3[:, 0] ** 2 + x3[:, 1] ** 2
    n_out = y[:, 0] ** 2 + y[:, 1] ** 2
    assert np.allclose(n_out, n_in * conc ** 2, rtol=1e-5)


# ---- bf16 rounding (fast_common.hpp:14-20) -----------------------------------

def test_bf16_special_cases():
    f = np.array([1.0, -0.0, 0.0, np.inf, -np.inf, 3.4e38,
                  np.frombuffer(np.uint32(0x3F808000).tobytes(), np.float32)[0],  # tie -> even (down)
                  np.frombuffer(np.uint32(0x3F818000).tobytes(), np.float32)[0],  # tie -> even (up)
                  np.frombuffer(np.uint32(0x3F808001).tobytes(), np.float32)[0],  # above tie -> up
                  np.frombuffer(np.uint32(0x7F800001).tobytes(), np.float32)[0],  # sNaN -> quiet
                  np.frombuffer(np.uint32(0x7F7FFFFF).tobytes(), np.float32)[0]],  # max -> inf
                 np.float32)
    want = [0x3F80, 0x8000, 0x0000, 0x7F80, 0xFF80, 0x7F80,  # 3.4e38: past the midpoint -> inf
            0x3F80, 0x3F82, 0x3F81, 0x7FC0, 0x7F80]
    got = O.to_bf16(f)
    for g, w in zip(got, want):
        assert g == w, (hex(g), hex(w))


def test_bf16_rne_sampled_exhaustive():
    # every upper half with a spread of lower halves, vs a float64 rounding
    hi = np.arange(0, 1 << 16, dtype=np.uint32)
    lows = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF, 0x1234, 0xC000], np.uint32)
    u = (hi[:, None] << 16 | lows[None, :]).reshape(-1)
    f = u.view(np.float32)
    finite = np.isfinite(f)
    got = O.to_bf16(f[finite]).astype(np.uint32)
    # reference rounding on magnitudes: nearest of the two bf16 neighbours,
    # ties to the even one; the neighbour above the largest finite is 2^128
    # (encoded 0x7F80 = inf), so overflow comes out of the same rule
    uf = u[finite]
    sign = (uf >> 16) & 0x8000
    m = (uf >> 16) & 0x7FFF
    e = (m >> 7).astype(np.int64)
    ulp = np.ldexp(1.0, np.where(e == 0, -133, e - 134).astype(np.int64))
    cand_lo = (m << 16).view(np.float32).astype(np.float64)
    a = np.abs(f[finite].astype(np.float64))
    d_lo, d_hi = a - cand_lo, cand_lo + ulp - a
    up = (d_hi < d_lo) | ((d_hi == d_lo) & (m % 2 == 1))
    want = sign | (m + up.astype(np.uint32))
    assert np.array_equal(got, want)
    nans = O.to_bf16(f[np.isnan(f)])
    assert np.all((nans & 0x7FFF) > 0x7F80) and np.all(nans & 0x40)


# ---- softmax and attention (run.cpp:335-353, 597-642) ------------------------

def test_softmax_matches_golden(golden):
    for row_in, row_out in zip(golden["softmax_in"], golden["softmax_out"]):
        assert np.array_equal(bits(O.softmax(row_in)), bits(row_out))


def _golden_cases(golden):
    for i in range(int(golden["n_cases"][0])):
        p = f"case{i}_"
        yield {k[len(p):]: golden[k] for k in golden.files if k.startswith(p)}


def test_decode_matches_reference_forward(golden):
    """The oracle reproduces run.cpp forward()'s attention output and the
    rotated key it writes, bit for bit, on full and window layers."""
    c, s = O.rope_table(4097)
    n = 0
    for case in _golden_cases(golden):
        hq, hkv, pos, W = (int(x) for x in case["meta"])
        q_rot, k_rot, _, _ = O.kv_append(case["qkv"][None], hq, hkv, c, s, [pos])
        kh = O.from_bf16(case["k_hist_bf16"]).reshape(pos, hkv, 64)
        vh = O.from_bf16(case["v_hist_bf16"]).reshape(pos, hkv, 64)
        v_new = case["qkv"][(hq + hkv) * 64:].reshape(1, hkv, 64)
        kc = np.concatenate([kh, k_rot])[None]
        vc = np.concatenate([vh, v_new])[None]
        for tag, window in (("full", 0), ("win", W)):
            assert np.array_equal(bits(k_rot[0]), bits(case["k_rot_" + tag]))
            out = O.decode_attention(q_rot, kc, vc, [pos], case["sinks"], window=window)
            assert np.array_equal(bits(out[0]), bits(case["out_" + tag])), (hq, pos, tag)
            n += 1
    assert n == 2 * int(golden["n_cases"][0])


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("hq,hkv", [(8, 2), (64, 8)])
def test_decode_matches_reference_build_random(hq, hkv):
    """Random cases straight through the reference build of run.cpp."""
    rng = np.random.default_rng(hq)
    c, s = O.rope_table(700)
    for pos in (2, 64, 129, 257, 600):
        row = (rng.standard_normal((hq + 2 * hkv) * 64) * 2).astype(np.float32)
        kh = rng.standard_normal((pos, hkv * 64)).astype(np.float32)
        vh = rng.standard_normal((pos, hkv * 64)).astype(np.float32)
        sinks = (rng.standard_normal(hq) * 2).astype(np.float32)
        q_rot, k_rot, _, _ = O.kv_append(row[None], hq, hkv, c, s, [pos])
        kc = np.concatenate([kh.reshape(pos, hkv, 64), k_rot])[None]
        vc = np.concatenate([vh.reshape(pos, hkv, 64), row[(hq + hkv) * 64:].reshape(1, hkv, 64)])[None]
        for wl in (False, True):
            ref_out, ref_k = O.ref_decode_one(row, kh, vh, sinks, pos, hq, hkv, window=128,
                                              window_layer=wl)
            out = O.decode_attention(q_rot, kc, vc, [pos], sinks, window=128 if wl else 0)
            assert np.array_equal(bits(out[0]), bits(ref_out))
            assert np.array_equal(bits(k_rot[0]), bits(ref_k))


@pytest.mark.skipif(not O.ref_available(), reason="oracle/_ref not built (needs /root/reference)")
def test_rope_and_softmax_match_reference_build():
    rng = np.random.default_rng(11)
    for p in (0, 1, 333, 4096, 9000):
        rc, rs = O.ref_cos_sin(p)
        c, s = O.rope_table(p + 1)
        assert np.array_equal(bits(c[p]), bits(rc)) and np.array_equal(bits(s[p]), bits(rs))
        x = (rng.standard_normal(8 * 64) * 4).astype(np.float32)
        assert np.array_equal(bits(O.rotate(x, c[p], s[p])), bits(O.ref_rotate(x, c[p], s[p])))
    for scale in (0.1, 1, 30, 200):
        x = (rng.standard_normal(1000) * scale).astype(np.float32)
        assert np.array_equal(bits(O.softmax(x)), bits(O.ref_softmax(x)))


def _fp64_attention(q, k, v, sink):
    s = (k.astype(np.float64) @ q.astype(np.float64)) / 8.0
    m = max(s.max(), sink)
    e = np.exp(s - m)
    return (e @ v.astype(np.float64)) / (e.sum() + np.exp(sink - m))


def test_decode_closed_forms():
    rng = np.random.default_rng(5)
    B, hq, hkv = 3, 8, 2
    q = rng.standard_normal((B, hq, 64)).astype(np.float32)
    sinks = rng.standard_normal(hq).astype(np.float32)
    # (i) n = 1: out = v * sigmoid(s - sink)
    k1 = rng.standard_normal((B, 1, hkv, 64)).astype(np.float32)
    v1 = rng.standard_normal((B, 1, hkv, 64)).astype(np.float32)
    out = O.decode_attention(q, k1, v1, [0] * B, sinks)
    for b in range(B):
        for h in range(hq):
            s = float(q[b, h].astype(np.float64) @ k1[b, 0, h // 4].astype(np.float64)) / 8
            want = v1[b, 0, h // 4] / (1 + np.exp(sinks[h] - s))
            assert np.allclose(out[b, h], want, rtol=1e-5, atol=1e-6)
    # (ii) identical keys: out = (1 - p_sink) * mean(v)
    n = 50
    kk = np.repeat(rng.standard_normal((B, 1, hkv, 64)).astype(np.float32), n, axis=1)
    vv = rng.standard_normal((B, n, hkv, 64)).astype(np.float32)
    out = O.decode_attention(q, kk, vv, [n - 1] * B, sinks)
    for b in range(B):
        for h in range(hq):
            s = float(q[b, h].astype(np.float64) @ kk[b, 0, h // 4].astype(np.float64)) / 8
            p_sink = 1.0 / (1 + n * np.exp(s - sinks[h]))
            want = (1 - p_sink) * vv[b, :, h // 4].astype(np.float64).mean(0)
            assert np.allclose(out[b, h], want, rtol=1e-4, atol=1e-5)
    # (iii) sink -> -inf: textbook softmax attention; and a brute-force fp64 check
    kc = rng.standard_normal((B, 40, hkv, 64)).astype(np.float32)
    vc = rng.standard_normal((B, 40, hkv, 64)).astype(np.float32)
    out = O.decode_attention(q, kc, vc, [39, 10, 0], np.full(hq, -1e30, np.float32))
    for b, p in enumerate([39, 10, 0]):
        for h in range(hq):
            ref = _fp64_attention(q[b, h], kc[b, :p + 1, h // 4], vc[b, :p + 1, h // 4], -1e30)
            assert np.allclose(out[b, h], ref, rtol=1e-5, atol=1e-6)
    # (iv) slot permutation on a ring: window output independent of slot order
    ring = 16
    pos = [20, 30, 15]
    kr = rng.standard_normal((B, ring, hkv, 64)).astype(np.float32)
    vr = rng.standard_normal((B, ring, hkv, 64)).astype(np.float32)
    a = O.decode_attention(q, kr, vr, pos, sinks, window=ring, ring=ring)
    for b, p in enumerate(pos):
        t = np.arange(max(0, p - ring + 1), p + 1)
        ref = [_fp64_attention(q[b, h], kr[b, t % ring, h // 4], vr[b, t % ring, h // 4], sinks[h])
               for h in range(hq)]
        assert np.allclose(a[b], np.array(ref), rtol=1e-5, atol=1e-6)
    # (v) window >= n equals full
    f = O.decode_attention(q, kc, vc, [39, 10, 0], sinks)
    w = O.decode_attention(q, kc, vc, [39, 10, 0], sinks, window=128)
    assert np.array_equal(bits(f), bits(w))
    # (vi) GQA: equal queries in a group give equal outputs
    q2 = q.copy()
    q2[:, 1] = q2[:, 0]
    o2 = O.decode_attention(q2, kc, vc, [39, 10, 0], sinks * 0)
    assert np.array_equal(bits(o2[:, 0]), bits(o2[:, 1]))


def test_prefill_is_decode_at_every_position():
    rng = np.random.default_rng(9)
    hq, hkv = 8, 2
    lens = [5, 1, 37, 140]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = cu[-1]
    q = rng.standard_normal((T, hq, 64)).astype(np.float32)
    k = rng.standard_normal((T, hkv, 64)).astype(np.float32)
    v = rng.standard_normal((T, hkv, 64)).astype(np.float32)
    sinks = rng.standard_normal(hq).astype(np.float32)
    for window in (0, 128):
        out = O.prefill_attention(cu, q, k, v, sinks, window=window)
        for b, L in enumerate(lens):
            r0 = cu[b]
            kc = k[r0:r0 + L][None]
            vc = v[r0:r0 + L][None]
            for j in range(L):
                d = O.decode_attention(q[r0 + j][None], kc, vc, [j], sinks, window=window)
                assert np.array_equal(bits(d[0]), bits(out[r0 + j]))
        # brute force fp64 on the smallest prompt
        for j in range(lens[0]):
            for h in range(hq):
                ref = _fp64_attention(q[j, h], k[:j + 1, h // 4], v[:j + 1, h // 4], sinks[h])
                assert np.allclose(out[j, h], ref, rtol=1e-5, atol=1e-6)


def test_oracle_rejects_bad_arguments():
    q = np.zeros((1, 8, 64), np.float32)
    kc = np.zeros((1, 4, 2, 64), np.float32)
    with pytest.raises(ValueError):
        O.decode_attention(q, kc, kc, [10], np.zeros(8, np.float32))  # pos beyond cache
    with pytest.raises(ValueError):
        O.decode_attention(q, kc, kc, [-1], np.zeros(8, np.float32))


def test_quantize_v_closed_forms():
    """int8-V rule (fast_misc.hpp:74-84): codes of exact multiples of the
    step, the amax element at +-127, ties to even, the all-zero head."""
    step = np.float32(3.0) / np.float32(127.0)
    k = np.arange(-63, 64, 2, dtype=np.float32)            # 64 values, amax at +-63
    v = np.concatenate([k[:63], [127.0]]).astype(np.float32) * step
    codes, scales = O.quantize_v(v.reshape(1, 64))
    assert codes[0, -1] == 127 and np.isclose(scales[0], 3.0 / 127.0, rtol=1e-7)
    assert np.array_equal(codes[0, :63], k[:63].astype(np.int8))
    # amax = 127 makes the reciprocal exactly 1: x.5 values round to even
    v = np.zeros(64, np.float32)
    v[:6] = [127.0, 2.5, 3.5, -2.5, -3.5, 0.5]
    codes, scales = O.quantize_v(v.reshape(1, 64))
    assert list(codes[0, :6]) == [127, 2, 4, -2, -4, 0] and scales[0] == 1.0
    codes, scales = O.quantize_v(np.zeros((2, 64), np.float32))
    assert not codes.any() and not scales.any()
    v = np.zeros(64, np.float32)
    v[7] = -0.75
    codes, scales = O.quantize_v(v.reshape(1, 64))
    assert codes[0, 7] == -127 and scales[0] == np.float32(0.75) / np.float32(127.0)
    # dequantized values stay within half a step of the input
    rng = np.random.default_rng(5)
    v = (rng.standard_normal((16, 64)) * 0.5).astype(np.float32)
    codes, scales = O.quantize_v(v)
    assert (np.abs(O.dequantize_v(codes, scales) - v) <= 0.5001 * scales[:, None]).all()


@pytest.mark.skipif(not O.ref_q8_available(), reason="reference build absent")
def test_quantize_v_matches_reference_build():
    rng = np.random.default_rng(11)
    for trial in range(200):
        v = (rng.standard_normal(64) * rng.choice([1e-3, 0.5, 3.0, 1e4])).astype(np.float32)
        if trial % 17 == 0:
            v[:] = 0.0
        codes, scales = O.quantize_v(v.reshape(1, 64))
        rc, rs = O.ref_quantize_v(v)
        assert np.array_equal(codes[0], rc) and np.float32(scales[0]) == np.float32(rs)


# ---- e4m3 K/V cache (no reference counterpart) -------------------------------

def test_fp8_table_closed_forms():
    """The e4m3 format's fixed points: 1.0, the largest finite value, the
    smallest normal and subnormal, NaN, monotone codes and sign symmetry."""
    t = O.fp8_table()
    assert t[0x38] == 1.0 and t[0x7E] == 448.0 and t[0x08] == 2.0 ** -6
    assert t[0x01] == 2.0 ** -9 and t[0x00] == 0.0 and t[0x40] == 2.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    pos = t[:0x7F]
    assert (np.diff(pos) > 0).all()                # monotone in the code
    assert np.array_equal(t[0x80:0xFF], -pos)      # sign bit
    # within one binade 8 equal steps; subnormals continue the lowest one
    assert np.allclose(np.diff(t[0x08:0x10]), 2.0 ** -9)
    assert np.allclose(np.diff(t[0x00:0x09]), 2.0 ** -9)


def _nearest_even_fp8(v, t):
    """Brute force: the code whose value is nearest v, ties to the even code
    (of v's sign for zero)."""
    fin = np.array([c for c in range(256) if not np.isnan(t[c])])
    d = np.abs(t[fin].astype(np.float64) - float(v))
    cand = fin[d == d.min()]
    if len(cand) > 1:
        cand = [c for c in cand if c % 2 == 0 and bool(c & 0x80) == bool(np.signbit(v))] or cand
    return int(cand[0])


def test_quantize_fp8_is_nearest_even():
    """Every code against a brute-force search of the table: random heads over
    seven decades, every midpoint between neighbouring values (ties), and the
    clamp edge."""
    t = O.fp8_table()
    rng = np.random.default_rng(21)
    x = (rng.standard_normal((300, 64)) *
         rng.choice([1e-6, 1e-3, 0.05, 1.0, 40.0, 1e4], (300, 1))).astype(np.float32)
    codes, scales = O.quantize_fp8(x)
    amax = np.abs(x).max(1)
    assert np.array_equal(scales, (amax / np.float32(448.0)).astype(np.float32))
    inv = (np.float32(448.0) / amax.astype(np.float32)).astype(np.float32)
    c = np.clip((x * inv[:, None]).astype(np.float32), -448.0, 448.0)
    for i in range(0, 300, 3):
        for j in range(64):
            assert codes[i, j] == _nearest_even_fp8(c[i, j], t), (c[i, j], codes[i, j])
    # midpoints between neighbouring positive values, each scaled into a head
    # whose amax is 448 (inv = 1, so the value itself is rounded)
    pos = t[:0x7F].astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (pos[:-1] + pos[1:]) / 2)  # exact in fp32
    for k in range(0, len(mids), 63):
        chunk = mids[k:k + 63]
        head = np.zeros(64, np.float32)
        head[0] = 448.0
        head[1:1 + len(chunk)] = chunk * np.where(np.arange(len(chunk)) % 2, -1, 1)
        cc, sc = O.quantize_fp8(head.reshape(1, 64))
        assert sc[0] == np.float32(1.0)
        for j in range(64):
            assert cc[0, j] == _nearest_even_fp8(head[j], t), (head[j], cc[0, j])
    # the largest element of a head is exactly -448 here
    h = np.array([[3.0, -7.5] + [0.1] * 62], np.float32)
    cc, sc = O.quantize_fp8(h)
    assert cc[0, 1] == 0xFE and sc[0] == np.float32(7.5) / np.float32(448.0)
    inv = np.float32(448.0) / np.float32(7.5)
    assert cc[0, 0] == _nearest_even_fp8(np.float32(3.0) * inv, t)
    cc, sc = O.quantize_fp8(np.zeros((2, 64), np.float32))
    assert not cc.any() and not sc.any()
    # dequantized values stay within half a step of their binade
    v = (rng.standard_normal((50, 64)) * 3).astype(np.float32)
    cc, sc = O.quantize_fp8(v)
    err = np.abs(O.dequantize_fp8(cc, sc) - v)
    assert (err <= np.maximum(np.abs(v) * 2.0 ** -4, 2.0 ** -10 * sc[:, None]) * 1.0001).all()


# ---- orc_linear (QKV projection: run.cpp matmul + bias add) ----------------

def _bf16_values(a):
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return u.view(np.float32)


def test_linear_matches_reference_matmul(oracle):
    """Bit-exact against run.cpp's own matmul + bias add (oracle/_ref)."""
    if not oracle.ref_available():
        pytest.skip("oracle/_ref not built (no reference sources)")
    rng = np.random.default_rng(21)
    x = _bf16_values(rng.standard_normal((4, 576)))
    w = _bf16_values(rng.standard_normal((320, 576)) * 0.05)
    b = (rng.standard_normal(320) * 0.1).astype(np.float32)
    got = oracle.linear(x, w, b)
    for r in range(4):
        ref = oracle.ref_matmul_bias(x[r], w, b)
        assert np.array_equal(got[r].view(np.uint32), ref.view(np.uint32))


def test_linear_closed_forms(oracle):
    """A one-hot row picks W's column exactly (plus the bias in fp32); with bf16
    inputs every product is exact, so the result is the fp64 sum rounded once
    to fp32, then the bias added in fp32."""
    rng = np.random.default_rng(22)
    n_in, n_out = 192, 128
    w = _bf16_values(rng.standard_normal((n_out, n_in)))
    b = rng.standard_normal(n_out).astype(np.float32)
    x = np.zeros((3, n_in), np.float32)
    x[0, 5] = 1.0
    x[1, 191] = -2.0
    x[2] = _bf16_values(rng.standard_normal(n_in))
    got = oracle.linear(x, w, b)
    assert np.array_equal(got[0], (w[:, 5] + b).astype(np.float32))
    assert np.array_equal(got[1], (np.float32(-2.0) * w[:, 191] + b).astype(np.float32))
    exact = (x[2].astype(np.float64) @ w.astype(np.float64).T).astype(np.float32) + b
    assert np.array_equal(got[2].view(np.uint32), exact.view(np.uint32))
    assert np.array_equal(oracle.linear(x, w, None)[0], w[:, 5])
