"""Pins the CPU oracle (oracle/zinc_oracle.c) before anything is compared to it.

Sources of truth, in order: the reference's own known-answer tests (values
copied from src/compute/forward.zig and forward_metal.zig test blocks), layout
statements the reference makes in comments (one set bit at a time must land on
the documented element), independent implementations (numpy float16, numpy
f64 matmul/softmax) and closed forms.
"""
import numpy as np
import pytest


def f16bits(v):
    return int(np.array(v, dtype=np.float16).view(np.uint16))


def put16(buf, off, v):
    b = f16bits(v)
    buf[off] = b & 0xFF
    buf[off + 1] = b >> 8


def pack_scale_min_k4(sc, m):
    """Inverse of getScaleMinK4 from its documented bit map (forward.zig:229-238):
    j<4: sc=s[j]&63, m=s[j+4]&63; j>=4: sc low nibble in s[j+4]&0xF, top 2 bits
    in s[j-4]>>6; m low nibble in s[j+4]>>4, top 2 bits in s[j]>>6."""
    s = [0] * 12
    for j in range(4):
        s[j] |= sc[j] & 63
        s[j + 4] |= m[j] & 63
    for j in range(4, 8):
        s[j + 4] |= (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (m[j] >> 4) << 6
    return np.array(s, dtype=np.uint8)


# ---------------------------------------------------------------- geometry
def test_block_geometry(orc):
    # gguf.zig:75-124
    assert (orc.block_size(orc.Q4_K), orc.bytes_per_block(orc.Q4_K)) == (256, 144)
    assert (orc.block_size(orc.Q6_K), orc.bytes_per_block(orc.Q6_K)) == (256, 210)
    assert (orc.block_size(orc.Q5_K), orc.bytes_per_block(orc.Q5_K)) == (256, 176)
    assert (orc.block_size(orc.Q8_0), orc.bytes_per_block(orc.Q8_0)) == (32, 34)
    assert (orc.block_size(orc.MXFP4), orc.bytes_per_block(orc.MXFP4)) == (32, 17)
    # forward.zig:11410-11416 expertSliceBytes KAT: Q4_K 512x2048 -> 589,824
    assert orc.tensor_bytes(orc.Q4_K, 512, 2048) == 589_824
    # BASELINE config 1 weight bytes
    assert orc.tensor_bytes(orc.Q4_K, 4096, 4096) == 9_437_184
    assert orc.tensor_bytes(orc.Q6_K, 151936, 4096) == 510_504_960


# ---------------------------------------------------------------- fp16
def test_f16_widen_all_patterns_match_numpy(orc):
    allh = np.arange(65536, dtype=np.uint16)
    ref = allh.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(h) for h in range(65536)], dtype=np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))
    assert np.array_equal(np.isinf(got), np.isinf(ref))


def test_f16_narrow_rne_matches_numpy(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.02),
        rng.standard_normal(20000).astype(np.float32) * 1000,
        (rng.standard_normal(5000) * 1e-6).astype(np.float32),  # subnormal range
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, -1e9, 2.0**-25, 2.0**-24,
                  1.5 * 2.0**-25, 2.0**-14, 6.1e-5], dtype=np.float32)])
    # halfway cases: f16 value + half ulp
    h = rng.integers(0, 0x7BFF, 5000).astype(np.uint16)
    base = h.view(np.float16).astype(np.float32)
    nxt = (h + 1).view(np.float16).astype(np.float32)
    vals = np.concatenate([vals, ((base.astype(np.float64) + nxt) / 2).astype(np.float32)])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.f32_to_f16(v) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- Q4_K
def test_get_scale_min_k4_kats(orc):
    # forward.zig:11590-11599
    s = np.zeros(12, np.uint8)
    s[0], s[4] = 0xFF, 0xC5
    assert orc.get_scale_min_k4(0, s) == (63, 5)
    # forward.zig:11601-11614
    s = np.zeros(12, np.uint8)
    s[0], s[4], s[8] = 0xC0, 0x80, 0x72
    assert orc.get_scale_min_k4(4, s) == (50, 39)


def test_get_scale_min_k4_roundtrip_every_field(orc):
    rng = np.random.default_rng(1)
    for _ in range(300):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        s = pack_scale_min_k4(sc, m)
        for j in range(8):
            assert orc.get_scale_min_k4(j, s) == (sc[j], m[j])


def test_dequant_q4k_kat_subblock_pairing(orc):
    # forward.zig:11465-11497
    blk = np.zeros(144, np.uint8)
    put16(blk, 0, 1.0)
    blk[4], blk[8], blk[5], blk[9] = 1, 0, 2, 0
    blk[16], blk[17] = 0x53, 0x97
    out = orc.dequant_row(blk, 0, 256, orc.Q4_K)
    assert abs(out[0] - 3.0) < 0.01 and abs(out[1] - 7.0) < 0.01
    assert abs(out[32] - 10.0) < 0.01 and abs(out[33] - 18.0) < 0.01


def test_dequant_q4k_single_bit_layout(orc):
    """d=1, every sc=1, dmin=0: setting bit k of qs byte b must produce exactly
    2^(k%4) at element 64*(b//32) + 32*(k//4) + b%32 (low nibbles of 32 bytes
    first, then their high nibbles; forward.zig:391-405 comment)."""
    for b in range(128):
        for k in range(8):
            blk = np.zeros(144, np.uint8)
            put16(blk, 0, 1.0)
            blk[4:16] = pack_scale_min_k4([1] * 8, [0] * 8)
            blk[16 + b] = 1 << k
            out = orc.dequant_row(blk, 0, 256, orc.Q4_K)
            exp = np.zeros(256, np.float32)
            exp[64 * (b // 32) + 32 * (k // 4) + b % 32] = 2 ** (k % 4)
            assert np.array_equal(out, exp), (b, k)


def test_dequant_q4k_closed_form_scales_and_mins(orc):
    """Uniform nibble q everywhere: sub-block j holds d*sc_j*q - dmin*m_j."""
    rng = np.random.default_rng(3)
    for _ in range(50):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = int(rng.integers(0, 16))
        d, dmin = np.float16(rng.random() * 0.05), np.float16(rng.random() * 0.05)
        blk = np.zeros(144, np.uint8)
        put16(blk, 0, d)
        put16(blk, 2, dmin)
        blk[4:16] = pack_scale_min_k4(sc, m)
        blk[16:] = q | (q << 4)
        out = orc.dequant_row(blk, 0, 256, orc.Q4_K)
        for j in range(8):
            v = np.float32(np.float32(d) * np.float32(sc[j])) * np.float32(q) - \
                np.float32(np.float32(dmin) * np.float32(m[j]))
            assert np.all(out[32 * j:32 * j + 32] == np.float32(v)), j


# ---------------------------------------------------------------- Q5_K
def test_dequant_q5k_kat_contiguous_halves(orc):
    # forward.zig:11499-11527: d=1, sc0=sc1=1, qh=0, qs[0]=0x3A -> out[0]=10, out[32]=3
    blk = np.zeros(176, np.uint8)
    put16(blk, 0, 1.0)
    blk[4], blk[5] = 1, 1
    blk[48] = 0x3A
    out = orc.dequant_row(blk, 0, 256, orc.Q5_K)
    assert abs(out[0] - 10.0) < 0.01 and abs(out[32] - 3.0) < 0.01


def test_dequant_q5k_single_bit_layout(orc):
    """d=1, every sc=1, dmin=0. A qs bit lands where Q4_K's does (element
    64*(b//32) + 32*(k//4) + b%32, value 2^(k%4)); bit k of qh[l] is the fifth
    bit (16) of element 32*k + l (ggml's dequantize_row_q5_K: bit 2p / 2p+1
    of qh[l] for the low / high half of 64-group p)."""
    def base():
        blk = np.zeros(176, np.uint8)
        put16(blk, 0, 1.0)
        blk[4:16] = pack_scale_min_k4([1] * 8, [0] * 8)
        return blk
    for b in range(128):
        for k in range(8):
            blk = base()
            blk[48 + b] = 1 << k
            exp = np.zeros(256, np.float32)
            exp[64 * (b // 32) + 32 * (k // 4) + b % 32] = 2 ** (k % 4)
            assert np.array_equal(orc.dequant_row(blk, 0, 256, orc.Q5_K), exp), ("qs", b, k)
    for l in range(32):
        for k in range(8):
            blk = base()
            blk[16 + l] = 1 << k
            exp = np.zeros(256, np.float32)
            exp[32 * k + l] = 16.0
            assert np.array_equal(orc.dequant_row(blk, 0, 256, orc.Q5_K), exp), ("qh", l, k)


def test_dequant_q5k_reduces_to_q4k(orc):
    """With qh = 0 a Q5_K block is the Q4_K block of the same header and qs;
    with qh = 0xFF every element gains d*sc_j*16 (exactly, in f32 for these
    small scales)."""
    rng = np.random.default_rng(21)
    for _ in range(20):
        b5 = rng.integers(0, 256, 176).astype(np.uint8)
        put16(b5, 0, np.float16(rng.random() * 0.05))
        put16(b5, 2, np.float16(rng.random() * 0.05))
        b4 = np.concatenate([b5[:16], b5[48:]])
        b5[16:48] = 0
        assert np.array_equal(orc.dequant_row(b5, 0, 256, orc.Q5_K), orc.dequant_row(b4, 0, 256, orc.Q4_K))
    for _ in range(20):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        q = int(rng.integers(0, 16))
        d, dmin = np.float16(rng.random() * 0.05), np.float16(rng.random() * 0.05)
        blk = np.zeros(176, np.uint8)
        put16(blk, 0, d)
        put16(blk, 2, dmin)
        blk[4:16] = pack_scale_min_k4(sc, m)
        blk[16:48] = 0xFF
        blk[48:] = q | (q << 4)
        out = orc.dequant_row(blk, 0, 256, orc.Q5_K)
        for j in range(8):
            v = np.float32(np.float32(d) * np.float32(sc[j])) * np.float32(q + 16) - \
                np.float32(np.float32(dmin) * np.float32(m[j]))
            assert np.all(out[32 * j:32 * j + 32] == np.float32(v)), j


def test_centered_q5k_model_init_is_zero_mean(orc):
    W = orc.synth_tensor(orc.Q5_K | 0x100, 64, 4096, 3, 4)
    w = orc.dequant(W, 64, 4096, orc.Q5_K).astype(np.float64)
    blk = W.reshape(-1, 176)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    dm = blk[:, 2:4].copy().view(np.float16).astype(np.float64).ravel()
    assert np.allclose(dm, (d * 15.5).astype(np.float16), rtol=0)
    assert abs(w.mean()) < 0.02 * np.abs(w).mean()
    # the header bytes follow the Q4_K generator's stream layout
    W4 = orc.synth_tensor(orc.Q4_K, 8, 256, 3, 4).reshape(-1, 144)
    W5 = orc.synth_tensor(orc.Q5_K, 8, 256, 3, 4).reshape(-1, 176)
    assert np.array_equal(W4[:, :144], W5[:, :144])


# ---------------------------------------------------------------- Q6_K
def _q6_block(d=1.0):
    blk = np.zeros(210, np.uint8)
    blk[192:208] = 1  # every int8 scale = 1
    put16(blk, 208, d)
    return blk


def test_dequant_q6k_single_bit_layout(orc):
    """GGML Q6_K layout (forward.zig:276-325 and dmmv_q6k.comp:122-137 agree):
    element e of half h=e//128, r=e%128, quarter g=r//32, l=r%32 takes its low
    4 bits from ql[64h + l + 32*(g&1)] (nibble g>>1) and its top 2 bits from
    qh[32h + l] bits 2g..2g+1; value d*sc[8h + l//16 + 2g]*(q-32)."""
    base = orc.dequant_row(_q6_block(), 0, 256, orc.Q6_K)
    assert np.all(base == -32.0)
    for b in range(128):
        for k in range(8):
            blk = _q6_block()
            blk[b] = 1 << k
            out = orc.dequant_row(blk, 0, 256, orc.Q6_K)
            h, lq = b // 64, b % 64
            g = (lq // 32) + 2 * (k // 4)
            e = 128 * h + 32 * g + lq % 32
            exp = np.full(256, -32.0, np.float32)
            exp[e] += 2 ** (k % 4)
            assert np.array_equal(out, exp), ("ql", b, k)
    for b in range(64):
        for k in range(8):
            blk = _q6_block()
            blk[128 + b] = 1 << k
            out = orc.dequant_row(blk, 0, 256, orc.Q6_K)
            h, l, g = b // 32, b % 32, k // 2
            exp = np.full(256, -32.0, np.float32)
            exp[128 * h + 32 * g + l] += 16 * 2 ** (k % 2)
            assert np.array_equal(out, exp), ("qh", b, k)


def test_dequant_q6k_scale_mapping(orc):
    for s in range(16):
        blk = _q6_block()
        blk[192 + s] = 3
        out = orc.dequant_row(blk, 0, 256, orc.Q6_K)
        exp = np.full(256, -32.0, np.float32)
        h, rem = s // 8, s % 8
        g, half16 = rem // 2, rem % 2
        lo = 128 * h + 32 * g + 16 * half16
        exp[lo:lo + 16] = -96.0
        assert np.array_equal(out, exp), s


def test_dequant_q6k_signed_scale_closed_form(orc):
    blk = _q6_block(0.5)
    blk[192:208] = np.array([-32, 31, -1, 5] * 4, dtype=np.int8).view(np.uint8)
    blk[0:128] = 0xFF   # low 4 bits all ones
    blk[128:192] = 0xFF  # high 2 bits all ones -> q = 63 -> q-32 = 31
    out = orc.dequant_row(blk, 0, 256, orc.Q6_K)
    sc = blk[192:208].view(np.int8)
    for e in range(256):
        h, r = e // 128, e % 128
        g, l = r // 32, r % 32
        s = sc[8 * h + l // 16 + 2 * g]
        assert out[e] == np.float32(np.float32(0.5) * np.float32(s)) * np.float32(31)


# ---------------------------------------------------------------- Q8_0
def test_dequant_q8_0_kat(orc):
    # forward.zig:11529-11553
    blk = np.zeros(34, np.uint8)
    put16(blk, 0, 0.5)
    blk[2:6] = np.array([1, -1, 127, -128], dtype=np.int8).view(np.uint8)
    out = orc.dequant_row(blk, 0, 32, orc.Q8_0)
    assert np.allclose(out[:4], [0.5, -0.5, 63.5, -64.0], atol=1e-3)
    assert out[6] == 0.0


def test_dot_q8_0_row_matches_dequant_dot(orc):
    # forward_metal.zig:12328 (dotQ8_0Row vs dequant + dot)
    rng = np.random.default_rng(5)
    K = 4096
    W = orc.synth_tensor(orc.Q8_0, 8, K, 11, 1)
    x = rng.standard_normal(K).astype(np.float32)
    y = orc.dmmv(W, orc.Q8_0, x, 8, K)
    ref = orc.dequant(W, 8, K, orc.Q8_0).astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-4, atol=1e-4)


# ---------------------------------------------------------------- F16 / F32
def test_dequant_f16_f32_kats(orc):
    # forward.zig:11555-11588
    raw = np.array([1.5, -3.25, 0.0, 42.0], np.float16).view(np.uint8)
    assert list(orc.dequant_row(raw, 0, 4, orc.F16)) == [1.5, -3.25, 0.0, 42.0]
    raw = np.array([1.0, -2.0, 3.14, 0.0], np.float32).view(np.uint8)
    assert np.array_equal(orc.dequant_row(raw, 0, 4, orc.F32), np.array([1.0, -2.0, 3.14, 0.0], np.float32))


# ---------------------------------------------------------------- MXFP4
def test_dequant_mxfp4_kat_and_specials(orc):
    # forward_metal.zig:14238-14303: e=127, every byte 0x42, x=1 -> 16*(1+2) = 48
    W = np.zeros(4 * 17, np.uint8)
    for r in range(4):
        W[r * 17] = 127
        W[r * 17 + 1:r * 17 + 17] = 0x42
    y = orc.dmmv(W, orc.MXFP4, np.ones(32, np.float32), 4, 32)
    assert np.all(y == 48.0)
    # e == 0 -> 2^-127 (bits 0x00400000, forward.zig:451); nibble 8 -> -0
    blk = np.zeros(17, np.uint8)
    blk[1] = 0x87  # lo = 7 (6.0), hi = 8 (-0)
    out = orc.dequant_row(blk, 0, 32, orc.MXFP4)
    assert out[0] == np.float32(6.0 * 2.0 ** -127)
    assert out[16] == 0.0 and np.signbit(out[16])
    # every code against E2M1 decoded from its bits: sign | exp(2) | man(1)
    for code in range(16):
        s, e, mbit = code >> 3, (code >> 1) & 3, code & 1
        mag = (mbit * 0.5) if e == 0 else (1 + 0.5 * mbit) * 2.0 ** (e - 1)
        blk = np.zeros(17, np.uint8)
        blk[0] = 130  # 2^3
        blk[1] = code
        out = orc.dequant_row(blk, 0, 32, orc.MXFP4)
        assert out[0] == np.float32((-1) ** s * mag * 8.0)


# ---------------------------------------------------------------- DMMV
@pytest.mark.parametrize("qtype,M,K", [(12, 64, 4096), (13, 64, 4096), (14, 64, 4096), (8, 64, 4096), (39, 64, 2880)])
def test_dmmv_matches_independent_f64(orc, qtype, M, K):
    W = orc.synth_tensor(qtype, M, K, 1234, 7)
    x = orc.synth_normal_f32(K, 1234, 99)
    y = orc.dmmv(W, qtype, x, M, K)
    ref = orc.dequant(W, M, K, qtype).astype(np.float64) @ x.astype(np.float64)
    mag = np.abs(orc.dequant(W, M, K, qtype).astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - ref) <= 1e-5 * mag + 1e-6)
    assert np.allclose(orc.dmmv_f64(W, qtype, x, M, K), ref, rtol=1e-12, atol=1e-9)
    assert np.allclose(orc.dmmv_absdot(W, qtype, x, M, K), mag, rtol=1e-12)
    # acc_mode 1: y += W x
    y0 = np.arange(M, dtype=np.float32)
    y1 = orc.dmmv(W, qtype, x, M, K, y=y0.copy(), acc_mode=1)
    assert np.array_equal(y1, (y0 + y).astype(np.float32)) or np.allclose(y1, y0 + y, rtol=1e-6)


# ---------------------------------------------------------------- elementwise
def test_rms_norm_closed_form_and_numpy(orc):
    n = 4096
    x = np.full(n, 3.0, np.float32)
    w = np.full(n, 2.0, np.float32)
    out = orc.rms_norm_mul(x, w, n, 1, 1e-6)
    assert np.allclose(out, 2.0 * 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-6)
    rng = np.random.default_rng(0)
    x = rng.standard_normal(2 * 128).astype(np.float32)
    w = rng.standard_normal(128).astype(np.float32)
    out = orc.rms_norm_mul(x, w, 128, 2, 1e-6)
    xr = x.reshape(2, 128).astype(np.float64)
    ref = (xr / np.sqrt((xr ** 2).mean(1, keepdims=True) + 1e-6)) * w
    assert np.allclose(out, ref.ravel(), rtol=1e-5, atol=1e-6)
    ph = orc.per_head_rms_norm(x, w, 128, 2, 1e-6)
    assert np.allclose(ph, ref.ravel(), rtol=1e-5, atol=1e-6)


def test_rope_identity_rotation_and_norm(orc):
    rng = np.random.default_rng(1)
    inv = orc.rope_inv_freq(128, 1e6)
    # forward.zig:1495-1500: 1/base^(2k/d)
    assert np.allclose(inv, 1.0 / (1e6 ** (np.arange(64) * 2 / 128)), rtol=1e-6)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    assert np.array_equal(orc.rope(x, 128, 128, 4, 0, inv), x)  # pos 0 = identity
    pos = 4100
    y = orc.rope(x, 128, 128, 4, pos, inv)
    xr = x.reshape(4, 128).astype(np.float64)
    th = pos * inv.astype(np.float64)
    # NeoX pairs (i, i+64)
    lo = xr[:, :64] * np.cos(th) - xr[:, 64:] * np.sin(th)
    hi = xr[:, :64] * np.sin(th) + xr[:, 64:] * np.cos(th)
    assert np.allclose(y.reshape(4, 128), np.concatenate([lo, hi], 1), atol=2e-3)
    assert np.allclose(np.hypot(y.reshape(4, 128)[:, :64], y.reshape(4, 128)[:, 64:]),
                       np.hypot(xr[:, :64], xr[:, 64:]), rtol=1e-5)


def test_swiglu_numpy(orc):
    rng = np.random.default_rng(2)
    g = rng.standard_normal(1000).astype(np.float32) * 5
    u = rng.standard_normal(1000).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(orc.swiglu(g, u), ref, rtol=1e-5, atol=1e-6)


def test_attention_seq1_returns_v_and_numpy(orc):
    rng = np.random.default_rng(4)
    hd, nh, nkv = 128, 32, 8
    q = rng.standard_normal(nh * hd).astype(np.float32)
    # seq_len=1 -> output == V (forward.zig:5224-5226 self-check)
    k = rng.standard_normal(nkv * hd).astype(np.float16).view(np.uint16)
    v = rng.standard_normal(nkv * hd).astype(np.float16).view(np.uint16)
    out = orc.attention_f16(q, k, v, hd, nh, nkv, 1)
    vf = v.view(np.float16).astype(np.float32).reshape(nkv, hd)
    assert np.array_equal(out.reshape(nh, hd), np.repeat(vf, nh // nkv, axis=0))
    L = 300
    k = rng.standard_normal(L * nkv * hd).astype(np.float16)
    v = rng.standard_normal(L * nkv * hd).astype(np.float16)
    out = orc.attention_f16(q, k.view(np.uint16), v.view(np.uint16), hd, nh, nkv, L)
    K = k.astype(np.float64).reshape(L, nkv, hd)
    V = v.astype(np.float64).reshape(L, nkv, hd)
    Q = q.astype(np.float64).reshape(nh, hd)
    ref = np.empty((nh, hd))
    for h in range(nh):
        s = K[:, h // 4, :] @ Q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h] = p @ V[:, h // 4, :]
    assert np.allclose(out, ref.ravel(), rtol=1e-4, atol=1e-5)


# ---------------------------------------------------------------- routing / sampling
def test_topk_softmax_kats(orc):
    # forward.zig:11392-11407
    ids, w = orc.topk_softmax([1.0, 3.0, 0.5, 2.0, 4.0, 1.5, 0.1, 0.2], 3)
    assert list(ids) == [4, 1, 3] and abs(w.sum() - 1) < 0.01 and w[0] > w[1] > w[2]
    # :11620-11629 uniform -> equal
    ids, w = orc.topk_softmax([1.0] * 4, 2)
    assert np.allclose(w, 0.5, atol=0.01)
    # :11631-11656 selected-only renormalised softmax
    lg = np.array([-2.0, 1.5, 0.25, 4.0, -0.5, 3.0, 2.5, -1.0], np.float32)
    ids, w = orc.topk_softmax(lg, 4)
    e = np.exp(lg[ids] - lg[ids].max())
    assert np.allclose(w, e / e.sum(), atol=1e-6)
    # :11658-11665 k=1
    ids, w = orc.topk_softmax([-1.0, 5.0, 2.0], 1)
    assert ids[0] == 1 and abs(w[0] - 1) < 1e-3
    # :11667-11680 large spread
    ids, w = orc.topk_softmax([100.0, 0.0, -100.0], 2)
    assert list(ids) == [0, 1] and w[0] > 0.99 and abs(w.sum() - 1) < 1e-3


def test_argmax_first_max_wins(orc):
    # forward.zig:11432-11437 and :10348-10356 (strict >, lowest index on ties)
    assert orc.argmax([0.5, 2.0, 1.25]) == 1
    assert orc.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert orc.argmax([-5.0, -5.0]) == 0


def test_kv_paging_kats(orc):
    import ctypes as C
    L = orc.lib()
    # forward.zig:11917-11923
    assert [L.zo_kv_page_count(n) for n in (0, 1, 16, 17, 4096)] == [0, 1, 1, 2, 256]
    # forward.zig:11931-11938
    pages = np.array([3, 1, 4], np.uint32)
    pp = pages.ctypes.data_as(C.POINTER(C.c_uint32))
    got = [L.zo_logical_to_physical(pp, 3, t) for t in (0, 15, 16, 18, 32)]
    assert got == [48, 63, 16, 18, 64]
    assert L.zo_logical_to_physical(pp, 3, 48) == -1  # ContextLengthExceeded


# ---------------------------------------------------------------- synthetic data
def test_synthetic_distributions(orc):
    W = orc.synth_tensor(orc.Q4_K, 256, 4096, 1, 2).reshape(-1, 144)
    d = W[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
    assert np.all(d >= 0) and abs(d.mean() - 0.02 * np.sqrt(2 / np.pi)) < 1e-3
    q = W[:, 16:]
    assert abs((q & 0xF).mean() - 7.5) < 0.05 and abs((q >> 4).mean() - 7.5) < 0.05
    W6 = orc.synth_tensor(orc.Q6_K, 64, 4096, 1, 3).reshape(-1, 210)
    sc = W6[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    W8 = orc.synth_tensor(orc.Q8_0, 64, 4096, 1, 4).reshape(-1, 34)
    qq = W8[:, 2:].view(np.int8)
    assert qq.min() == -127 and qq.max() == 127
    Wm = orc.synth_tensor(orc.MXFP4, 64, 2880, 1, 5).reshape(-1, 17)
    assert Wm[:, 0].min() == 118 and Wm[:, 0].max() == 130
    z = orc.synth_normal_f32(200000, 1, 6)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    # determinism and stream separation
    assert np.array_equal(orc.synth_tensor(orc.Q4_K, 4, 256, 1, 2), W[:4].ravel())
    assert not np.array_equal(orc.synth_tensor(orc.Q4_K, 4, 256, 1, 9), W[:4].ravel())


def test_centered_q4k_model_init_is_zero_mean(orc):
    """The model-init variant (dmin = f16(7.5 d)) removes the positive mean of
    BASELINE-distributed Q4_K weights, so mat-vec outputs have no common mode."""
    W0 = orc.synth_tensor(orc.Q4_K, 64, 4096, 3, 4)
    W1 = orc.synth_tensor(orc.Q4_K | 0x100, 64, 4096, 3, 4)
    d0, d1 = orc.dequant(W0, 64, 4096, orc.Q4_K), orc.dequant(W1, 64, 4096, orc.Q4_K)
    assert d0.mean() > 1.0                      # BASELINE blocks: strongly positive mean
    assert abs(d1.mean()) < 0.02 * d1.std()     # centered
    b = W1.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dm = b[:, 2:4].copy().view(np.float16).ravel()
    assert np.array_equal(dm, (d * np.float32(7.5)).astype(np.float16))
    assert np.array_equal(b[:, 4:], W0.reshape(-1, 144)[:, 4:])  # scales and codes unchanged


def test_more_bits_rule_counts(orc):
    # llama.cpp's use_more_bits: the first and last eighth of the layers and
    # every third layer between, i.e. half of a 32-layer model's attn_v /
    # ffn_down (the Q4_K_M mix of 7B-class GGUF files: layers 0-3, 6, 9, ..,
    # 27, 28-31)
    L = orc.lib()
    sel32 = [i for i in range(32) if L.zo_more_bits_layer(i, 32)]
    assert sel32 == [0, 1, 2, 3, 6, 9, 12, 15, 18, 21, 24, 27, 28, 29, 30, 31]
    sel36 = [i for i in range(36) if L.zo_more_bits_layer(i, 36)]
    assert sel36[:4] == [0, 1, 2, 3] and sel36[-5:] == [31, 32, 33, 34, 35] and len(sel36) == 18


def test_model_set_tensor_matches_more_bits_config(orc):
    """A model whose more_bits layers were replaced tensor by tensor decodes
    exactly as the model built with type_more_bits (same bytes, same types)."""
    base = dict(n_layers=8, hidden=256, n_heads=2, n_kv_heads=1, head_dim=128, ffn=512, vocab=300,
                n_experts=0, n_experts_used=0, expert_ffn=0, max_ctx=64, type_attn=12, type_ffn_gate_up=12,
                type_ffn_down=12, type_lm_head=14, type_embd=12, type_router=8, rope_base=1e6, eps=1e-6, seed=5)
    a = orc.Model(dict(base, type_more_bits=14), nthreads=4)
    b = orc.Model(base, nthreads=4)
    for l in (0, 3, 6, 7):
        for kind, shape in ((orc.K_WV, (128, 256)), (orc.K_DOWN, (256, 512))):
            s = orc.S_LAYER(l, kind)
            assert a.tensor_type(s) == 14 and b.tensor_type(s) == 12
            b.set_tensor(s, 14, orc.synth_tensor(14 | 0x100, *shape, base["seed"], s))
            assert np.array_equal(a.tensor(s), b.tensor(s))
    assert a.tensor_type(orc.S_LAYER(1, orc.K_WV)) == 12
    with pytest.raises(ValueError):
        b.set_tensor(orc.S_LAYER(1, orc.K_WV), 14, np.zeros(10, np.uint8))
    for pos, tok in enumerate((3, 7, 11)):
        ta, la = a.decode_step(tok, pos, want_logits=True)
        tb, lb = b.decode_step(tok, pos, want_logits=True)
        assert ta == tb and np.array_equal(la, lb)
    a.close()
    b.close()


# ---- sampleFromLogits (forward.zig:10261-10334) ----------------------------
def test_sampling_reference_cases(orc):
    # forward.zig:11425-11459
    L = orc.lib()
    assert not L.zo_sampling_requires_readback(0.0, 1.0, 1.0)
    assert L.zo_sampling_requires_readback(0.7, 1.0, 1.0)
    assert L.zo_sampling_requires_readback(0.0, 0.9, 1.0)
    assert L.zo_sampling_requires_readback(0.0, 1.0, 1.1)
    assert orc.sample_from_logits([0.5, 2.0, 1.25], u=0.3) == 1
    assert orc.sample_from_logits([10.0, 9.0, 1.0], [0, 0, 0], temperature=0.0, repetition_penalty=2.0) == 1
    for u in (0.0, 0.3, 0.97):
        assert orc.sample_from_logits([8.0, 5.0, 1.0], temperature=0.8, top_p=0.5, top_k=8, u=u) == 0
    # the top_p scan stops only past the first candidate (forward.zig:10311),
    # so two candidates stay: the second (share exp(-3.75) / (1 + exp(-3.75))
    # = 0.0230) takes the top of the draw
    assert orc.sample_from_logits([8.0, 5.0, 1.0], temperature=0.8, top_p=0.5, top_k=8, u=0.99) == 1


def _support_and_freq(orc, logits, n_u=20000, **kw):
    us = (np.arange(n_u) + 0.5) / n_u
    toks = np.array([orc.sample_from_logits(logits, u=float(u), **kw) for u in us])
    ids, cnt = np.unique(toks, return_counts=True)
    return dict(zip(ids.tolist(), (cnt / n_u).tolist()))


def test_sampling_distribution_is_topk_softmax(orc):
    rng = np.random.default_rng(0)
    lg = rng.normal(0, 2, 300).astype(np.float32)
    T, k = 0.7, 12
    freq = _support_and_freq(orc, lg, temperature=T, top_k=k)
    top = np.argsort(-lg, kind="stable")[:k]
    assert set(freq) == set(top.tolist())
    z = lg[top].astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    for t, pt in zip(top.tolist(), p):
        assert abs(freq[t] - pt) < 2e-4, (t, freq[t], pt)


def test_sampling_top_p_support_is_minimal_prefix(orc):
    rng = np.random.default_rng(1)
    lg = rng.normal(0, 1.5, 200).astype(np.float32)
    T, k, tp = 1.0, 40, 0.6
    freq = _support_and_freq(orc, lg, temperature=T, top_k=k, top_p=tp)
    top = np.argsort(-lg, kind="stable")[:k]
    z = lg[top].astype(np.float64) / T
    p = np.exp(z - z.max())
    p /= p.sum()
    # shortest prefix with cumulative share >= top_p, at least two candidates
    keep = max(int(np.searchsorted(np.cumsum(p), tp) + 1), 2)
    assert set(freq) == set(top[:keep].tolist())
    q = p[:keep] / p[:keep].sum()
    for t, pt in zip(top[:keep].tolist(), q):
        assert abs(freq[t] - pt) < 2e-4


def test_sampling_ties_nonfinite_and_penalty(orc):
    # equal logits at the top-k boundary: the earlier token is kept
    lg = np.array([1.0, 3.0, 2.0, 2.0, 2.0], np.float32)
    assert set(_support_and_freq(orc, lg, n_u=2000, temperature=1.0, top_k=2)) == {1, 2}
    # non-finite logits never become candidates when sampling ...
    lg = np.array([np.nan, 1.0, np.inf, 0.5, -np.inf], np.float32)
    assert set(_support_and_freq(orc, lg, n_u=2000, temperature=1.0, top_k=8)) == {1, 3}
    # ... but the greedy scan compares them: +inf wins, a NaN at index 0 stays
    assert orc.sample_from_logits(lg, repetition_penalty=1.5, temperature=0.0) == 0
    assert orc.sample_from_logits(np.array([0.0, np.inf, 1.0], np.float32), top_p=0.5, temperature=0.0) == 1
    # penalty: positive seen logits shrink (/p), negative ones grow (*p)
    assert orc.sample_from_logits(np.array([4.0, 2.5], np.float32), [0], temperature=0.0,
                                  repetition_penalty=2.0) == 1
    assert orc.sample_from_logits(np.array([-1.0, -1.5], np.float32), [0], temperature=0.0,
                                  repetition_penalty=2.0) == 1
    assert orc.sample_from_logits(np.array([-1.0, -2.5], np.float32), [0], temperature=0.0,
                                  repetition_penalty=2.0) == 0
    # a single finite candidate is returned whatever u is
    assert orc.sample_from_logits(np.array([np.nan, 7.0, np.nan], np.float32), temperature=0.9, u=0.99) == 1


def test_dequant_q4k_f32_tie_block(orc):
    """d = 293/2048, dmin = 2^-24 (the smallest fp16 subnormal), every sc and
    m = 1, every q = 7: dj*q - mj = 2051/2048 - 2^-24 lies halfway between two
    f32 values and rounds to the even one, 2051/2048 -- itself halfway between
    fp16 1 + 2^-10 and 1 + 2^-9, which rounds to 1 + 2^-9. (The GPU prefill
    GEMM's fp16 operand test uses this block: rounding the exact value to
    fp16 once would give 1 + 2^-10.)"""
    blk = np.zeros(144, np.uint8)
    put16(blk, 0, np.float16(293 / 2048))
    blk[2:4] = np.array([1], np.uint16).view(np.uint8)
    blk[4:16] = pack_scale_min_k4([1] * 8, [1] * 8)
    assert list(blk[4:16]) == [1] * 8 + [0x11] * 4
    blk[16:] = 0x77
    out = orc.dequant_row(blk, 0, 256, orc.Q4_K)
    assert np.all(out == np.float32(2051 / 2048))
    assert np.all(out.astype(np.float16) == np.float16(1 + 2 ** -9))
