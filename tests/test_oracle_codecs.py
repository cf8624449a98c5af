"""Pins of the CPU oracle's codecs and ops against facts fixed independently of it:
IEEE binary16 (numpy), the GGML block layouts written out as a vectorised numpy
closed form, f64 brute force, and closed-form identities."""
import numpy as np
import pytest

import oracle_py as O

rng = np.random.default_rng(1234)


# ---------------------------------------------------------------- fp16
def test_fp16_to_fp32_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([O.oracle().orc_fp16_to_fp32(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_fp32_to_fp16_round_nearest_even():
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-8, 5, 20000),
                        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 1 + 2 ** -11, 1 + 3 * 2 ** -11],
                                 dtype=np.float32)]).astype(np.float32)
    ref = x.astype(np.float16).view(np.uint16)
    got = np.array([O.oracle().orc_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- independent closed forms
def f16(raw2):
    return np.frombuffer(bytes(raw2), dtype=np.float16).astype(np.float32)[0]


def q4k_closed_form(raw):
    """block_q4_K: {f16 d, f16 dmin, u8 scales[12], u8 qs[128]}; 8 sub-blocks of 32 with 6-bit
    scale / min; y = (d*sc)*q - dmin*m in float32 with one rounding per operation."""
    b = np.frombuffer(bytes(raw), dtype=np.uint8).reshape(-1, 144)
    out = []
    for blk in b:
        d, dmin = f16(blk[0:2]), f16(blk[2:4])
        s = blk[4:16].astype(np.int32)
        sc = np.zeros(8, np.int32)
        mn = np.zeros(8, np.int32)
        sc[:4], mn[:4] = s[:4] & 63, s[4:8] & 63
        sc[4:] = (s[8:12] & 15) | ((s[0:4] >> 6) << 4)
        mn[4:] = (s[8:12] >> 4) | ((s[4:8] >> 6) << 4)
        qs = blk[16:].reshape(4, 32).astype(np.int32)
        q = np.stack([qs & 15, qs >> 4], axis=1).reshape(256)          # group g: low then high nibbles
        sub = np.arange(256) // 32
        a = (np.float32(d) * sc[sub].astype(np.float32)).astype(np.float32)
        m = (np.float32(dmin) * mn[sub].astype(np.float32)).astype(np.float32)
        out.append((a * q.astype(np.float32)).astype(np.float32) - m)
    return np.concatenate(out).astype(np.float32)


def q6k_closed_form(raw):
    """block_q6_K: {u8 ql[128], u8 qh[64], i8 scales[16], f16 d}; q = 4 low bits | 2 high bits << 4,
    minus 32; 16 sub-blocks of 16; y = (d*sc)*q."""
    b = np.frombuffer(bytes(raw), dtype=np.uint8).reshape(-1, 210)
    out = []
    for blk in b:
        ql = blk[0:128].astype(np.int32).reshape(2, 2, 32)   # [half][first/second 32][l]
        qh = blk[128:192].astype(np.int32).reshape(2, 32)
        sc = blk[192:208].view(np.int8).astype(np.float32)
        d = f16(blk[208:210])
        q = np.zeros((2, 4, 32), np.int32)
        for quarter in range(4):
            low = ql[:, quarter & 1, :]
            low = (low & 15) if quarter < 2 else (low >> 4)
            q[:, quarter, :] = low | (((qh >> (2 * quarter)) & 3) << 4)
        q = q.reshape(256) - 32
        a = (np.float32(d) * sc[np.arange(256) // 16]).astype(np.float32)
        out.append((a * q.astype(np.float32)).astype(np.float32))
    return np.concatenate(out)


def q80_closed_form(raw):
    b = np.frombuffer(bytes(raw), dtype=np.uint8).reshape(-1, 34)
    return np.concatenate([blk[2:].view(np.int8).astype(np.float32) * f16(blk[:2]) for blk in b]).astype(np.float32)


def _f16bytes(v):
    return np.array([v], dtype=np.float16).tobytes()


def handbuilt_q4k():
    """Blocks covering every 6-bit scale and min value in every sub-block slot, every nibble,
    and d/dmin that are normal, subnormal, negative and zero."""
    blocks = []
    ds = [(0.013, 0.004), (6.1e-5, 3.0e-7), (-0.5, 0.25), (0.0, 0.1), (1.0, 0.0), (2.0 ** -14, 2.0 ** -24)]
    for bi in range(64):
        d, dmin = ds[bi % len(ds)]
        sc = [(bi + 8 * j) % 64 for j in range(8)]
        mn = [(63 - bi + 5 * j) % 64 for j in range(8)]
        s = np.zeros(12, np.uint8)
        for j in range(4):
            s[j] = sc[j] & 63
            s[j + 4] = mn[j] & 63
        for j in range(4, 8):
            s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
        qs = ((np.arange(128) * 7 + bi) % 16) | ((((np.arange(128) * 3 + 5 * bi) % 16)) << 4)
        blocks.append(_f16bytes(d) + _f16bytes(dmin) + s.tobytes() + qs.astype(np.uint8).tobytes())
    return b"".join(blocks)


def handbuilt_q6k():
    blocks = []
    for bi in range(16):
        ql = ((np.arange(128) * 5 + bi) % 256).astype(np.uint8)
        qh = ((np.arange(64) * 37 + 3 * bi) % 256).astype(np.uint8)
        sc = np.array([((bi * 16 + j) * 17) % 256 - 128 for j in range(16)], dtype=np.int8)
        d = [0.0021, -0.75, 6.0e-8, 0.0, 3.0][bi % 5]
        blocks.append(ql.tobytes() + qh.tobytes() + sc.tobytes() + _f16bytes(d))
    return b"".join(blocks)


def handbuilt_q80():
    blocks = []
    for bi in range(8):
        qs = np.array([((bi * 32 + j) * 11) % 256 - 128 for j in range(32)], dtype=np.int8)
        d = [0.01, -3.5, 1e-6, 0.0, 1.0, 65504.0, 2.0 ** -24, 0.3333][bi]
        blocks.append(_f16bytes(d) + qs.tobytes())
    return b"".join(blocks)


def test_q4k_handbuilt_covers_every_value():
    raw = handbuilt_q4k()
    b = np.frombuffer(raw, np.uint8).reshape(-1, 144)
    nib = np.concatenate([b[:, 16:] & 15, b[:, 16:] >> 4], axis=None)
    assert set(nib.tolist()) == set(range(16))


@pytest.mark.parametrize("name,typ,build,closed,n_per", [
    ("q4_K", O.Q4_K, handbuilt_q4k, q4k_closed_form, 256),
    ("q6_K", O.Q6_K, handbuilt_q6k, q6k_closed_form, 256),
    ("q8_0", O.Q8_0, handbuilt_q80, q80_closed_form, 32),
])
def test_dequant_matches_closed_form(name, typ, build, closed, n_per):
    raw = build()
    n = len(raw) // O.BLOCK[typ][1] * n_per
    got = O.dequant(typ, np.frombuffer(raw, np.uint8), n)
    ref = closed(raw)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name


def test_dequant_random_bytes_q4k_q6k():
    # random blocks with finite d (exponent field < 31)
    for typ, size, dpos, closed in ((O.Q4_K, 144, (0, 2), q4k_closed_form), (O.Q6_K, 210, (208,), q6k_closed_form)):
        raw = rng.integers(0, 256, size * 50, dtype=np.uint8).reshape(50, size)
        for p in dpos:
            raw[:, p + 1] &= 0x7B   # clear exponent MSB -> finite f16
        got = O.dequant(typ, raw.reshape(-1), 50 * 256)
        assert np.array_equal(got.view(np.uint32), closed(raw.tobytes()).view(np.uint32))


# ---------------------------------------------------------------- activation quantisation
def test_q8K_roundtrip_and_special_cases():
    x = (rng.standard_normal(256 * 20) * 10.0 ** rng.integers(-3, 3, 256 * 20)).astype(np.float32)
    x[:256] = 0.0                                   # all-zero block
    x[256:512] = np.linspace(-1, 1, 256, dtype=np.float32)
    raw = O.quantize_q8_K(x)
    blk = np.frombuffer(raw.tobytes(), dtype=np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bs", "<i2", 16)]))
    assert blk["d"][0] == 0 and not blk["qs"][0].any()
    for i in range(1, 20):
        xb = x[256 * i:256 * (i + 1)]
        d, q = blk["d"][i], blk["qs"][i].astype(np.int32)
        j = int(np.argmax(np.abs(xb)))             # first index of max |x|
        assert q[j] == -127                         # iscale = -127/max maps the max to -127
        assert np.all(np.abs(xb - d * q) <= abs(d) * 0.5 * (1 + 1e-5) + 1e-30)
        assert np.array_equal(blk["bs"][i], q.reshape(16, 16).sum(1))
    deq = O.dequant(O.Q8_K, raw, x.size)
    assert np.allclose(deq, x, rtol=0, atol=np.max(np.abs(x)) / 127)


def test_q80_act_roundtrip():
    x = rng.standard_normal(32 * 40).astype(np.float32)
    raw = O.quantize_q8_0(x)
    blk = np.frombuffer(raw.tobytes(), dtype=np.dtype([("d", "<f2"), ("qs", "i1", 32)]))
    for i in range(40):
        xb = x[32 * i:32 * (i + 1)]
        d = np.abs(xb).max() / 127
        assert np.all(np.abs(blk["qs"][i].astype(np.int32)) <= 127)
        # q = roundf(x/d) with the unrounded d; stored d is f16(d)
        assert np.array_equal(blk["qs"][i], np.sign(xb / d) * np.floor(np.abs(xb / d) + 0.5))


# ---------------------------------------------------------------- vec_dot / mul_mat vs f64 brute force
def random_weights(typ, rows, cols):
    import dfx
    x = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    return dfx.quantize_rows(typ, x)


@pytest.mark.parametrize("typ", [O.Q4_K, O.Q6_K, O.Q8_0, O.F16])
def test_mul_mat_matches_f64_bruteforce(typ):
    N, K, M = 16, 768, 5
    W = random_weights(typ, N, K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    Y = O.mul_mat(typ, W, N, K, X)
    Wf = np.stack([O.dequant(typ, W[n * O.row_bytes(typ, K):(n + 1) * O.row_bytes(typ, K)], K) for n in range(N)])
    Xc = O.act_convert(typ, X)        # the activation values the dot products see
    ref = Xc.astype(np.float64) @ Wf.astype(np.float64).T
    assert np.max(np.abs(Y - ref)) <= 2e-5 * np.max(np.abs(ref))
    # a plausible mistake (dot against unconverted activations) is visibly different for K-quants
    if typ in (O.Q4_K, O.Q6_K):
        wrong = X.astype(np.float64) @ Wf.astype(np.float64).T
        assert np.max(np.abs(wrong - ref)) > 10 * np.max(np.abs(Y - ref))


# ---------------------------------------------------------------- rms_norm / rope / silu
def test_rms_norm_closed_form():
    x = rng.standard_normal((7, 512)).astype(np.float32) * 3
    w = rng.standard_normal(512).astype(np.float32)
    y = O.rms_norm_mul(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-6)) < 1e-5


def test_rope_table_closed_form():
    hd, base, n_pos = 128, 500000.0, 800
    tab = O.rope_table(n_pos, hd, base).reshape(n_pos, hd // 2, 2)
    p = np.arange(n_pos)[:, None].astype(np.float64)
    i = np.arange(hd // 2)[None, :].astype(np.float64)
    theta = p * base ** (-2 * i / hd)
    assert np.max(np.abs(tab[..., 0] - np.cos(theta))) < 2e-3
    assert np.max(np.abs(tab[..., 1] - np.sin(theta))) < 2e-3
    assert np.array_equal(tab[0, :, 0], np.ones(hd // 2, np.float32))    # position 0: identity


def test_rope_neox_rotates_half_pairs():
    import ctypes as C
    hd, H, M = 128, 3, 5
    x = rng.standard_normal((M, H, hd)).astype(np.float32)
    pos = np.array([0, 1, 7, 100, 300], dtype=np.int32)
    tab = O.rope_table(301, hd, 10000.0)
    y = x.copy()
    O.oracle().orc_rope_neox(O.ptr(y), M, H, hd, O.ptr(pos), O.ptr(tab))
    assert np.array_equal(y[0], x[0])
    t = tab.reshape(301, hd // 2, 2)[pos]            # [M][half][cos,sin]
    c, s = t[:, None, :, 0].astype(np.float64), t[:, None, :, 1].astype(np.float64)
    x0, x1 = x[..., :hd // 2].astype(np.float64), x[..., hd // 2:].astype(np.float64)
    assert np.allclose(y[..., :hd // 2], x0 * c - x1 * s, atol=1e-5)
    assert np.allclose(y[..., hd // 2:], x0 * s + x1 * c, atol=1e-5)
    assert np.allclose(np.hypot(y[..., :hd // 2], y[..., hd // 2:]), np.hypot(x0, x1), rtol=1e-5)


@pytest.mark.parametrize("M,n_keys,H,Hkv,hd", [(5, 37, 4, 4, 128), (9, 64, 8, 2, 64)])
def test_attention_bruteforce_and_invariances(M, n_keys, H, Hkv, hd):
    """f64 brute force of softmax(q k^T / sqrt(hd)) v with head h reading KV head
    h // (H/Hkv); the result is invariant (bitwise) to the order of the keys."""
    r = np.random.default_rng(7)
    q = r.standard_normal((M, H, hd)).astype(np.float32) * 2
    k = r.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    v = r.standard_normal((n_keys, Hkv, hd)).astype(np.float32)
    got = O.attention(q, k, v)
    rep = H // Hkv
    kd, vd = np.repeat(k.astype(np.float64), rep, 1), np.repeat(v.astype(np.float64), rep, 1)
    s = np.einsum("mhd,nhd->hmn", q.astype(np.float64), kd) / np.sqrt(hd)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = np.einsum("hmn,nhd->mhd", p, vd)
    assert np.abs(got - ref).max() < 1e-5 * np.abs(ref).max()
    perm = r.permutation(n_keys)
    assert np.array_equal(O.attention(q, k[perm], v[perm]), got)
    # one dominant key: the output is (almost) that key's value row
    q1 = q[:1, ::rep].repeat(rep, axis=1)            # heads of one KV group share the query
    k2 = k.copy()
    k2[3] = q1[0, ::rep] * 50
    assert np.allclose(O.attention(q1, k2, v)[0], np.repeat(v[3], rep, 0), atol=1e-4)


def test_silu():
    for v in (-20.0, -1.0, 0.0, 0.5, 3.0, 30.0):
        assert abs(O.oracle().orc_silu(v) - v / (1 + np.exp(-v))) < 1e-6 * max(1, abs(v))


# ---------------------------------------------------------------- sampler pieces
# Sequences the cosine / linear formulas give when each step's count is unmasked.
COSINE_256_16 = [1, 4, 6, 8, 11, 13, 15, 17, 19, 20, 22, 23, 23, 24, 25, 25]
COSINE_64_16 = [1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 5, 5, 6, 6, 6, 6]


@pytest.mark.parametrize("B,schedule,expect", [(256, 0, COSINE_256_16), (64, 0, COSINE_64_16), (256, 1, [16] * 16)])
def test_schedule_sequences(B, schedule, expect):
    masked, seq = B, []
    for step in range(16):
        n = O.tokens_to_unmask(step, 16, masked, schedule)
        seq.append(n)
        masked -= n
    assert seq == expect and sum(seq) == B


def seq_f32_entropy(x):
    """The reference's float32 sequence (src/diffuse-sampler.cpp:34-57): running float sums
    in index order (np.cumsum on float32 is sequential), p > 1e-10 filter."""
    x = np.asarray(x, np.float32)
    mx = x.max()
    s = np.cumsum(np.exp(x - mx).astype(np.float32), dtype=np.float32)[-1]
    lp = ((x - mx) - np.float32(np.log(s))).astype(np.float32)
    p = np.exp(lp).astype(np.float32)
    t = np.where(p > np.float32(1e-10), -(p * lp), np.float32(0)).astype(np.float32)
    return float(np.cumsum(t, dtype=np.float32)[-1])


def test_entropy_special_rows():
    V = 126464
    u = np.zeros(V, np.float32)
    # sequential float accumulation loses ~1e-3 relative on a uniform 126464-row (swamping)
    assert abs(O.entropy(u) - seq_f32_entropy(u)) < 1e-5
    assert abs(O.entropy(u) - np.log(V)) < 2e-3 * np.log(V)
    one_hot = np.full(V, -100.0, np.float32)
    one_hot[123] = 100.0
    assert abs(O.entropy(one_hot)) < 1e-6
    two = np.full(1000, -1e4, np.float32)
    two[[3, 900]] = 5.0
    assert abs(O.entropy(two) - np.log(2)) < 1e-6
    x = rng.standard_normal(5000).astype(np.float32) * 2
    p = np.exp(x.astype(np.float64) - x.max())
    p /= p.sum()
    assert abs(O.entropy(x) - float(-(p * np.log(p)).sum())) < 1e-4


def test_top2_semantics():
    assert O.top2(np.array([5, 5, 1], np.float32)) == (0, 5.0, 5.0)            # tie -> lowest index
    assert O.top2(np.array([1, 7, 3, 7], np.float32)) == (1, 7.0, 7.0)
    assert O.top2(np.array([3, 7, 5], np.float32)) == (1, 7.0, 5.0)
    b, bv, sv = O.top2(np.array([2.0], np.float32))
    assert (b, bv) == (0, 2.0) and sv == np.float32(-1e30)
    for _ in range(50):
        x = rng.integers(-5, 5, 40).astype(np.float32)
        b, bv, sv = O.top2(x)
        assert b == int(np.argmax(x)) and bv == x.max()
        assert sv == (np.delete(x, b).max() if b > 0 else max(np.delete(x, b).max(), np.float32(-1e30)))


@pytest.mark.parametrize("remasking", [0, 2, 3, 4])
def test_order_candidates_bruteforce(remasking):
    for trial in range(20):
        n = int(rng.integers(1, 300))
        c = np.zeros(n, O.CAND)
        c["pos"] = rng.permutation(1000)[:n]
        c["token"] = rng.integers(0, 100, n)
        c["confidence"] = rng.integers(0, 10, n).astype(np.float32)     # many ties
        c["entropy"] = rng.integers(0, 6, n).astype(np.float32) * 0.5
        n_sched = int(rng.integers(1, n + 1))
        got, nu = O.order_candidates(c, remasking, 1.5, n_sched)
        if remasking == 2:
            key = sorted(range(n), key=lambda i: (c["entropy"][i], c["pos"][i]))
            expect_n = min(max(n_sched, int((c["entropy"] < 1.5).sum())), n)
        else:
            key = sorted(range(n), key=lambda i: (-c["confidence"][i], c["pos"][i]))
            expect_n = min(n_sched, n)
        assert np.array_equal(got["pos"], c["pos"][key])
        assert nu == expect_n
