"""Pins of the CPU oracle (CPU only).

The reference holds no golden vectors for the MoE path (its only numeric
check, `qe check`, needs real weights and llama.cpp).  Each oracle function is
pinned here by closed forms, special cases, brute force or an independent
restatement, chosen so a plausible slip (dropped term, wrong sign/index,
transposed operand, wrong rounding or tie rule) fails a check.
"""
import math
import os
import re

import numpy as np
import pytest

import oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KV = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.int64)
SEED = 0x5EED


def _header_consts():
    txt = open(os.path.join(REPO, "qe-qwen36-b50_amd", "csrc", "qe_format.h")).read()
    return {m[0]: int(m[1], 16) for m in re.findall(r"#define (QE_NL4_W\d) (0x[0-9A-Fa-f]+)u", txt)}


def test_codebook_words_match_reference_constants():
    w = _header_consts()
    packed = np.array(KV, np.int8).view(np.uint8).tobytes()
    assert [w["QE_NL4_W%d" % i] for i in range(4)] == list(np.frombuffer(packed, "<u4"))
    # engine/qe.cpp:78-79 packs the same table as two 64-bit constants
    assert (w["QE_NL4_W1"] << 32) | w["QE_NL4_W0"] == 0xF6EADDCFBFAD9881
    assert (w["QE_NL4_W3"] << 32) | w["QE_NL4_W2"] == 0x7159453526190D01


def test_row_and_blob_sizes():
    # engine/pack.h:28-42 closed forms
    assert 2048 // 2 + 2048 // 32 * 2 == 1152
    assert 512 // 2 + 512 // 32 * 2 == 288
    assert 2 * 512 * 1152 + 2048 * 288 == O.EXPERT_BYTES == 1769472
    assert O.SH_GU_BYTES == 1024 * (2048 + 128) and O.SH_DN_BYTES == 2048 * (512 + 32)
    assert len(O.gen_expert(SEED, 0, 0)) == 1769472


def test_f16_conversion_matches_ieee_rne():
    lib = O.load()
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.02),
        (rng.random(20000) * 2.0 ** rng.integers(-30, 17, 20000)).astype(np.float32),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e-8, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 0.0005], np.float32),
    ])
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in vals], np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    allh = np.arange(65536, dtype=np.uint16)
    fin = np.isfinite(allh.view(np.float16))
    back = np.array([lib.orc_f16_to_f32(int(h)) for h in allh[fin]], np.float32)
    assert np.array_equal(back.view(np.uint32), allh[fin].view(np.float16).astype(np.float32).view(np.uint32))


def test_log_and_cos_against_libm():
    lib = O.load()
    rng = np.random.default_rng(2)
    for u in list(rng.random(2000) + 1e-12) + [1.0, 2.0 ** -32, 0.5, math.sqrt(0.5)]:
        assert abs(lib.orc_log_unit(u) - math.log(u)) <= 4e-16 * max(1.0, abs(math.log(u)))
    for t in list(rng.random(2000)) + [0.0, 0.25, 0.5, 0.75, 0.999999]:
        assert abs(lib.orc_cos_turns(t) - math.cos(2 * math.pi * t)) <= 2e-15


def test_normal_moments():
    x = O.gen_x(SEED, 7, 64).reshape(-1).astype(np.float64)  # 131072 samples
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1.0) < 0.01
    assert abs(((x - x.mean()) ** 3).mean()) < 0.03 and abs((x ** 4).mean() - 3.0) < 0.06


def _quant_ref(x):
    """numpy restatement of quant_x (float32 arithmetic, round half to even)."""
    x = x.astype(np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d > 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.clip(np.rint(x * idv[:, None]), -128, 127).astype(np.int8)
    return q.reshape(-1), d


def test_quant_x_special_cases():
    z = np.zeros(32, np.float32)
    q, s = O.quant_x(z)
    assert s[0] == 0 and not q.any()
    x = np.zeros(32, np.float32)
    x[5] = -3.0
    q, s = O.quant_x(x)
    assert q[5] == -127 and np.count_nonzero(q) == 1 and s[0] == np.float32(3.0) / np.float32(127)
    # amax 127 -> d = 1 exactly: halves round to even
    x = np.array([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5] + [0] * 24, np.float32)
    q, s = O.quant_x(x)
    assert s[0] == 1.0 and list(q[:8]) == [127, 2, 4, -2, -4, 0, 0, 2]
    x = -x
    q, _ = O.quant_x(x)
    assert q[0] == -127


def test_quant_x_scalar_avx2_and_numpy_agree():
    rng = np.random.default_rng(3)
    for scale in (1.0, 1e-3, 1e4):
        x = (rng.standard_normal(2048) * scale).astype(np.float32)
        q1, s1 = O.quant_x(x)
        q2, s2 = O.quant_x(x, avx2=True)
        q3, s3 = _quant_ref(x)
        assert np.array_equal(q1, q2) and np.array_equal(q1, q3)
        assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32)) and np.array_equal(s1, s3)


def _decode_nl4_row(row, cols):
    codes = row[: cols // 2].reshape(-1, 16)
    lo, hi = codes & 15, codes >> 4
    idx = np.concatenate([lo, hi], axis=1).reshape(-1)  # element j<16 low nibble of byte j, j+16 high
    scales = row[cols // 2: cols // 2 + cols // 32 * 2].view(np.float16).astype(np.float64)
    return KV[idx], scales


def test_dot_nl4_brute_force_and_forms_agree():
    rng = np.random.default_rng(4)
    blob = O.gen_expert(SEED, 0, 3)
    for cols, off, rb in ((2048, 0, 1152), (2048, 700 * 1152, 1152), (512, 1179648 + 99 * 288, 288)):
        row = blob[off: off + rb]
        x = rng.standard_normal(cols).astype(np.float32)
        xq, xs = O.quant_x(x)
        a = O.dot_nl4(row, cols, xq, xs)
        b = O.dot_nl4(row, cols, xq, xs, avx2=True)
        assert np.float32(a).view(np.uint32) == np.float32(b).view(np.uint32)
        w, sc = _decode_nl4_row(row, cols)
        p = (w.reshape(-1, 32) * xq.astype(np.int64).reshape(-1, 32)).sum(axis=1)  # exact per-block int dots
        exact = float((sc * xs.astype(np.float64) * p).sum())
        assert abs(a - exact) <= 2e-6 * np.abs(sc * xs * p).sum()
    # a transposed nibble order (element j+16 taken from the low nibble) must not pass
    wrong = KV[np.concatenate([row[:256].reshape(-1, 16) >> 4, row[:256].reshape(-1, 16) & 15], 1).reshape(-1)]
    assert not np.array_equal(wrong, _decode_nl4_row(row, 512)[0])


def test_dot_nl4_x4_equals_single_token_dots():
    # the CPU baseline's 4-token form (weights decoded once per group, the
    # reference's cpu_dot_nl4_x4) gives each token the single-token result bit
    # for bit, for every group size 1..4 and both row lengths; a per-group
    # scale slip (token 0's xs used for all) must not pass
    rng = np.random.default_rng(41)
    blob = O.gen_expert(SEED, 1, 7)
    for cols, off, rb in ((2048, 5 * 1152, 1152), (512, 1179648 + 1000 * 288, 288)):
        row = blob[off: off + rb]
        xq, xs = zip(*[O.quant_x(rng.standard_normal(cols).astype(np.float32) * (1 + 3 * i)) for i in range(4)])
        for n in range(1, 5):
            got = O.dot_nl4_x4(row, cols, xq[:n], xs[:n])
            want = np.array([O.dot_nl4(row, cols, xq[i], xs[i], avx2=True) for i in range(n)], np.float32)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (cols, n)
        slip = O.dot_nl4_x4(row, cols, xq, [xs[0]] * 4)
        assert not np.array_equal(slip[1:].view(np.uint32), want[1:].view(np.uint32))


def test_canon_dot_and_rmsnorm():
    rng = np.random.default_rng(5)
    a = rng.standard_normal(2048).astype(np.float32)
    b = rng.standard_normal(2048).astype(np.float32)
    exact = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(O.canon_dot(a, b) - exact) <= 1e-5 * float(np.abs(a.astype(np.float64) * b).sum())
    # exactly representable case: every partial is an integer
    ai = rng.integers(-8, 8, 2048).astype(np.float32)
    assert O.canon_dot(ai, ai) == float((ai.astype(np.int64) ** 2).sum())
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    w = rng.random(2048).astype(np.float32) + 0.5
    xn = O.rmsnorm(x, w)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6) * w
    assert np.abs(xn - ref).max() <= 2e-6 * np.abs(ref).max()
    c = np.full((1, 2048), 3.0, np.float32)
    assert np.allclose(O.rmsnorm(c, np.ones(2048, np.float32)), 3.0 / math.sqrt(9.0 + 1e-6), rtol=1e-7)


def _sumsq_tree_f32(x):
    """float32 emulation of the canonical sum of squares for inputs with one
    non-zero element per group of 8 (the group's fma chain is then one rounded
    square): the pairwise tree over the 256 groups, adjacent pairs first."""
    p = (x.reshape(256, 8).astype(np.float32) ** 2).sum(axis=1, dtype=np.float32)
    s = 1
    while s < 256:
        p[0::2 * s] = p[0::2 * s] + p[s::2 * s]
        s *= 2
    return p[0]


def test_canon_sumsq_order():
    rng = np.random.default_rng(11)
    # small integers: every partial is exact, so any order gives the exact sum
    xi = rng.integers(-20, 20, 2048).astype(np.float32)
    assert O.canon_sumsq(xi) == float((xi.astype(np.int64) ** 2).sum())
    # one non-zero per group, random magnitudes: bit-exact against the tree emulation
    for trial in range(20):
        x = np.zeros(2048, np.float32)
        x[np.arange(256) * 8 + rng.integers(0, 8, 256)] = (rng.standard_normal(256) * 2.0 ** rng.integers(-6, 7, 256))
        assert np.float32(O.canon_sumsq(x)) == _sumsq_tree_f32(x), trial
    # adversarial: 2^24 in group 0 and 1 in every other group.  The tree loses only
    # group 1 (2^24 + 1 rounds to 2^24) and gives 2^24 + 254; a sequential sum
    # loses every 1, float64 keeps all
    x = np.zeros(2048, np.float32)
    x[0] = 4096.0
    x[8::8] = 1.0
    assert O.canon_sumsq(x) == 2.0 ** 24 + 254
    seq = np.float32(0)
    for v in (x.reshape(256, 8) ** 2).sum(axis=1, dtype=np.float32):
        seq = np.float32(seq + v)
    assert seq == 2.0 ** 24 and O.canon_sumsq(x) != seq
    # the norm uses it: xn = x / sqrt(ss / 2048 + eps) * w, elementwise in fp32
    w = (rng.random(2048) + 0.5).astype(np.float32)
    xr = rng.standard_normal(2048).astype(np.float32)
    inv = np.float32(1.0) / np.sqrt(np.float32(O.canon_sumsq(xr)) / np.float32(2048) + np.float32(1e-6), dtype=np.float32)
    assert np.array_equal(O.rmsnorm(xr[None], w)[0], (xr * inv) * w)


def _topk_ref(lg):
    """Closed form of engine/qe.cpp:1454-1483: order by (-value, e % 16, e // 16)."""
    e = np.arange(256)
    order = sorted(e, key=lambda i: (-float(lg[i]), i % 16, i // 16))
    return np.array(order[:8])


def test_topk_all_equal_and_ties():
    lg = np.zeros((1, 257), np.float32)
    ids, wts, shg = O.topk(lg)
    assert list(ids[0]) == [0, 16, 32, 48, 64, 80, 96, 112]
    assert np.allclose(wts, 0.125) and shg[0] == 0.5
    rng = np.random.default_rng(6)
    for trial in range(200):
        lg = rng.integers(-3, 3, size=257).astype(np.float32)  # many ties
        ids, _, _ = O.topk(lg[None])
        assert list(ids[0]) == list(_topk_ref(lg)), trial
    # -0.0 and +0.0 tie
    lg = np.full(257, -5.0, np.float32)
    lg[33], lg[2] = -0.0, 0.0
    ids, _, _ = O.topk(lg[None])
    assert list(ids[0][:2]) == [33, 2]  # 33 % 16 = 1 < 2 % 16 = 2


def test_topk_distinct_and_weights():
    rng = np.random.default_rng(7)
    lg = rng.standard_normal((64, 257)).astype(np.float32)
    ids, wts, shg = O.topk(lg)
    for t in range(64):
        want = np.argsort(-lg[t, :256], kind="stable")[:8]
        assert np.array_equal(ids[t], want)
        sel = lg[t, ids[t]].astype(np.float64)
        p = np.exp(sel - sel[0])
        assert np.allclose(wts[t], p / p.sum(), rtol=2e-6, atol=0)
        assert abs(shg[t] - 1 / (1 + math.exp(-float(lg[t, 256])))) < 1e-6


def test_dispatch_fixture_and_random():
    fx = np.load(os.path.join(REPO, "tests", "golden", "routing_records.npz"))
    names = sorted({k.rsplit("_", 1)[0] for k in fx.files})
    assert names
    for n in names:
        off, pairs = O.dispatch(fx[n + "_ids"].astype(np.int32))
        assert np.array_equal(off, fx[n + "_off"]) and np.array_equal(pairs, fx[n + "_pairs"])
    rng = np.random.default_rng(8)
    for T in (1, 7, 300):
        ids = np.stack([rng.choice(256, 8, replace=False) for _ in range(T)]).astype(np.int32)
        off, pairs = O.dispatch(ids)
        flat = ids.reshape(-1)
        assert np.array_equal(pairs, np.argsort(flat, kind="stable"))
        assert np.array_equal(np.diff(off), np.bincount(flat, minlength=256))


def _f64_layer(L, x, ids, wts, shg):
    """Independent float64 restatement of one layer from the raw bytes."""
    T = x.shape[0]
    out = np.zeros((T, 2048))
    sgu = L.sh_gu.reshape(1024, 2176)
    Wsh = sgu[:, :2048].view(np.int8).astype(np.float64) * np.repeat(sgu[:, 2048:].view(np.float16).astype(np.float64), 32, 1)
    sdn = L.sh_dn.reshape(2048, 544)
    Dsh = sdn[:, :512].view(np.int8).astype(np.float64) * np.repeat(sdn[:, 512:].view(np.float16).astype(np.float64), 32, 1)
    exps = L.experts(ids)
    for t in range(T):
        xq, xs = _quant_ref(x[t])
        xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
        g, u = Wsh[:512] @ x[t].astype(np.float64), Wsh[512:] @ x[t].astype(np.float64)
        hsh = g / (1 + np.exp(-g)) * u
        acc = shg[t] * (Dsh @ hsh)
        for k in range(8):
            blob = exps[int(ids[t, k])]
            rows = blob[:1179648].reshape(1024, 1152)
            W = np.stack([np.repeat(_decode_nl4_row(r, 2048)[1], 32) * _decode_nl4_row(r, 2048)[0] for r in rows])
            gu = W @ xd
            with np.errstate(over="ignore"):
                h = gu[:512] / (1 + np.exp(-gu[:512])) * gu[512:]
            hq, hs = _quant_ref(h.astype(np.float32))
            hd = hq.astype(np.float64) * np.repeat(hs.astype(np.float64), 32)
            drows = blob[1179648:].reshape(2048, 288)
            Dm = np.stack([np.repeat(_decode_nl4_row(r, 512)[1], 32) * _decode_nl4_row(r, 512)[0] for r in drows])
            acc = acc + wts[t, k] * (Dm @ hd)
        out[t] = acc
    return out


def test_full_layer_against_float64_restatement():
    L = O.SynthLayer(SEED, 0)
    x = O.gen_x(SEED, 1, 1)
    r = O.moe_layer(L, x)
    ref = _f64_layer(L, x, r["ids"], r["wts"].astype(np.float64), r["shg"].astype(np.float64))
    rel = np.linalg.norm(r["out"] - ref) / np.linalg.norm(ref)
    assert rel < 1e-4, rel
    # the shared-expert term on its own (it is ~1e-5 of the output norm)
    sgu = L.sh_gu.reshape(1024, 2176)
    Wsh = sgu[:, :2048].view(np.int8).astype(np.float64) * np.repeat(sgu[:, 2048:].view(np.float16).astype(np.float64), 32, 1)
    sdn = L.sh_dn.reshape(2048, 544)
    Dsh = sdn[:, :512].view(np.int8).astype(np.float64) * np.repeat(sdn[:, 512:].view(np.float16).astype(np.float64), 32, 1)
    g, u = Wsh[:512] @ x[0].astype(np.float64), Wsh[512:] @ x[0].astype(np.float64)
    sd = Dsh @ (g / (1 + np.exp(-g)) * u)
    assert np.linalg.norm(r["sd"][0] - sd) / np.linalg.norm(sd) < 1e-6


def _router_f64(xn, W, bias):
    """float64 logits of engine/qe.cpp:144-150 with the shared-gate row appended
    as row 256 (:1055): W[e] . xn for e = 0..256, bias on rows 0..255 only; and
    the sum of |terms|, which bounds any fp32 summation order's error."""
    xd, Wd = xn.astype(np.float64), W.astype(np.float64)
    lg, scale = xd @ Wd.T, np.abs(xd) @ np.abs(Wd).T
    if bias is not None:
        lg[:, :256] += bias.astype(np.float64)
        scale[:, :256] += np.abs(bias.astype(np.float64))
    return lg, scale


def _router_matches(lg32, xn, W, bias):
    ref, scale = _router_f64(xn, W, bias)
    return lg32.shape == ref.shape and bool(np.all(np.abs(lg32.astype(np.float64) - ref) <= 1e-5 * scale))


def test_router_against_float64():
    L = O.SynthLayer(SEED, 3)
    xn = O.rmsnorm(3.0 * O.gen_x(SEED, 21, 5), None)
    bias = (0.5 + np.random.default_rng(21).random(256)).astype(np.float32)  # no entry near 0
    for b in (None, bias):
        assert _router_matches(O.router(xn, L.router, b), xn, L.router, b)
    lg = O.router(xn, L.router, bias)
    # row 256 is a plain dot with the shared-gate vector, no bias
    g64 = xn.astype(np.float64) @ L.router[256].astype(np.float64)
    assert np.all(np.abs(lg[:, 256] - g64) <= 1e-5 * (np.abs(xn) @ np.abs(L.router[256]).astype(np.float64)))
    # planted slips fail the same check: bias also on row 256 (a loop to e <= 256
    # reading bias[e % 256]), bias dropped, rows off by one, bias on the wrong row
    bad = lg.copy()
    bad[:, 256] += bias[0]
    assert not _router_matches(bad, xn, L.router, bias)
    assert not _router_matches(O.router(xn, L.router, None), xn, L.router, bias)
    assert not _router_matches(O.router(xn, np.ascontiguousarray(np.roll(L.router, -1, 0)), bias), xn, L.router, bias)
    assert not _router_matches(O.router(xn, L.router, np.ascontiguousarray(np.roll(bias, 1))), xn, L.router, bias)


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_layer_wiring_norm_and_residual_against_float64():
    """moe_layer(norm, residual) is x + MoE(RMSNorm(x) * post_norm)
    (engine/qe.cpp:1958 entry norm, :2036-2044 combine onto the residual), with
    the norm, routing, weights and gate recomputed in float64 here."""
    L = O.SynthLayer(SEED, 4)
    # The MoE output does not depend on the input's scale (the norm removes it) and
    # is ~3e4 in rms with these synthetic weights; x at rms 1e4 keeps the residual
    # (and a skipped norm) visible at the 1e-4 bar.
    x = (1e4 * O.gen_x(SEED, 22, 2)).astype(np.float32)
    pn = (1.0 + 0.25 * O.gen_x(SEED, 23, 1)[0]).astype(np.float32)
    r = O.moe_layer(L, x, norm=True, residual=True, post_norm=pn)
    xd = x.astype(np.float64)
    xn64 = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + 1e-6) * pn.astype(np.float64)
    assert _rel(r["xn"], xn64) < 1e-6
    lg64, _ = _router_f64(xn64, L.router, None)
    ids64 = np.stack([_topk_ref(lg64[t]) for t in range(2)])
    assert np.array_equal(r["ids"], ids64)
    sel = np.take_along_axis(lg64[:, :256], ids64, axis=1)
    p = np.exp(sel - sel[:, :1])
    wts64 = p / p.sum(axis=1, keepdims=True)
    shg64 = 1.0 / (1.0 + np.exp(-lg64[:, 256]))
    moe64 = _f64_layer(L, xn64.astype(np.float32), ids64, wts64, shg64)
    ref = xd + moe64

    def ok(out):
        return _rel(out, ref) < 1e-4

    assert ok(r["out"])
    # planted wiring slips, each must fail: residual taken from the normed input,
    # no residual, the norm skipped, the norm weight dropped
    assert not ok(xn64 + moe64)
    assert not ok(r["out"] - xd)
    assert not ok(xd + O.moe_layer(L, x)["out"])
    assert not ok(xd + O.moe_layer(L, O.rmsnorm(x, None))["out"])


def test_scalar_and_avx2_layers_agree_bitwise():
    L = O.SynthLayer(SEED, 1, bias=O.gen_zipf_bias(SEED, 1, 1.0))
    x = O.gen_x(SEED, 2, 3)
    ids, wts, _ = O.topk(O.router(x, L.router, L.bias))
    ya = O.routed(x, ids, wts, L.experts(ids), avx2=True)
    ys = O.routed(x, ids, wts, L.experts(ids), avx2=False)
    assert np.array_equal(ya.view(np.uint32), ys.view(np.uint32))


def test_baseline_layer_matches_oracle():
    import ctypes
    L = O.SynthLayer(SEED, 2, bias=O.gen_zipf_bias(SEED, 2, 1.0))
    x = O.gen_x(SEED, 3, 4)
    r = O.moe_layer(L, x)
    exps = L.experts(r["ids"])
    ptrs = (ctypes.c_void_p * 256)()
    for e, b in exps.items():
        ptrs[e] = b.ctypes.data
    _, out = O.baseline_layer(x, None, L, ptrs, 4, 4)
    assert np.linalg.norm(out - r["out"]) / np.linalg.norm(r["out"]) < 1e-5
    # with norm + residual (config 2's layer)
    pn = np.ones(2048, np.float32)
    r2 = O.moe_layer(L, x, norm=True, residual=True)
    exps = L.experts(r2["ids"])
    for e, b in exps.items():
        ptrs[e] = b.ctypes.data
    _, out2 = O.baseline_layer(x, pn, L, ptrs, 4, 4)
    assert np.linalg.norm(out2 - r2["out"]) / np.linalg.norm(r2["out"]) < 1e-5


def test_zipf_bias_is_a_permutation_of_log_ranks():
    b = O.gen_zipf_bias(SEED, 0, 1.0)
    ranks = np.sort(np.round(np.exp(-b.astype(np.float64))).astype(int))
    assert np.array_equal(ranks, np.arange(1, 257))
    b13 = O.gen_zipf_bias(SEED, 0, 1.3)
    assert np.allclose(b13, 1.3 * b, rtol=1e-6)


# ---------------------------------------------------------------------------
# IQ4_NL converter (ggml's quantizer as engine/qconv.cpp:91-98 calls it)
# ---------------------------------------------------------------------------
def _nearest_brute(a):
    """Index of the codebook entry closest to each float32 a; equal distances go to the larger entry."""
    a = np.asarray(a, np.float32)
    dist = np.abs(a[:, None] - KV.astype(np.float32)[None, :])  # float32 differences, as ggml rounds them
    return 15 - np.argmin(dist[:, ::-1], axis=1)


def _nearest_mid(a):
    """Count of bracket midpoints <= a (the form the GPU kernel evaluates)."""
    mids = (KV[:-1] + KV[1:]).astype(np.float32) / np.float32(2)
    return np.sum(np.asarray(a, np.float32)[:, None] >= mids[None, :], axis=1)


def test_nl4_nearest_brute_force_and_midpoint_form():
    rng = np.random.default_rng(11)
    mids = (KV[:-1] + KV[1:]) / 2.0
    a = [rng.uniform(-160, 160, 20000), KV, mids, [0.0, -0.0, -127.0, 113.0, -1e6, 1e6, 1e-30, -1e-30]]
    near = [np.concatenate([np.asarray(v, np.float32) for v in a])]
    for v in np.concatenate([mids, KV]).astype(np.float32):  # a thousand ulps either side of each
        u = np.full(1001, v, np.float32)
        for i in range(1, 1001):
            u[i] = np.nextafter(u[i - 1], np.float32(np.inf))
        w = np.full(1001, v, np.float32)
        for i in range(1, 1001):
            w[i] = np.nextafter(w[i - 1], np.float32(-np.inf))
        near += [u, w]
    a = np.concatenate(near)
    got = np.array([O.nl4_nearest(float(v)) for v in a])
    assert np.array_equal(got, _nearest_brute(a))
    assert np.array_equal(got, _nearest_mid(a))
    # ties go to the larger entry: 7 is midway between 1 and 13
    assert O.nl4_nearest(7.0) == 9 and O.nl4_nearest(np.nextafter(np.float32(7), np.float32(0))) == 8


def _dequant_block(d16, codes):
    idx = np.concatenate([codes & 15, codes >> 4]).astype(np.int64)
    return KV[idx].astype(np.float64) * float(np.array([d16], np.uint16).view(np.float16)[0])


def test_nl4_block_exact_fit_recovers_scale_and_codes():
    rng = np.random.default_rng(12)
    for trial in range(200):
        s = np.float32(2.0 ** int(rng.integers(-12, 4))) * (1 if trial % 2 else -1)
        idx = rng.integers(0, 16, 32)
        idx[rng.integers(0, 32)] = 0  # -127: the entry of largest magnitude fixes m
        x = (KV[idx] * s).astype(np.float32)
        d16, codes, d = O.nl4_block(x)
        assert d == s and d16 == int(np.array([s], np.float16).view(np.uint16)[0])
        assert np.array_equal(np.concatenate([codes & 15, codes >> 4]), idx), trial  # byte j: j | j+16 << 4
        assert np.array_equal(_dequant_block(d16, codes), x.astype(np.float64))


def _candidates(x):
    """ggml's 16 candidate inverse scales of a block, in float32."""
    x = np.asarray(x, np.float32)
    j = int(np.argmax(np.abs(x)))  # first of the largest |x|
    m = x[j]
    s = [np.float32(1) / (m / np.float32(127))]
    s += [np.float32(t - 127) / m for t in range(-7, 8)]
    return s


def _objective(x, s):
    """Weighted least-squares fit of one candidate, in float64: (score, d)."""
    x64 = np.asarray(x, np.float64)
    q = KV[_nearest_brute(np.float32(s) * np.asarray(x, np.float32))].astype(np.float64)
    w = x64 * x64
    sxq, sqq = np.sum(w * q * x64), np.sum(w * q * q)
    return sxq * sxq / sqq, sxq / sqq


def test_nl4_block_picks_the_best_candidate():
    rng = np.random.default_rng(13)
    gens = [lambda: rng.standard_normal(32), lambda: rng.standard_t(3, 32), lambda: rng.uniform(-1, 1, 32),
            lambda: np.where(rng.random(32) < 0.2, rng.standard_normal(32) * 20, rng.standard_normal(32))]
    blocks = [gens[i % 4]() * 10.0 ** rng.uniform(-4, 2) for i in range(2000)]
    for b in blocks[::8]:  # +A and -A both present: m is the first of them
        j = int(np.argmax(np.abs(b)))
        b[(j + 1 + int(rng.integers(0, 31))) % 32] = -b[j]
    hist = np.zeros(16, int)
    for x in blocks:
        x = np.asarray(x, np.float32)
        d16, codes, d = O.nl4_block(x)
        objs = [_objective(x, s) for s in _candidates(x)]
        score = np.array([o[0] for o in objs])
        best = int(np.argmax(score))
        hist[best] += 1
        # the chosen fit is a best-scoring candidate's (near-ties within fp32 rounding)
        ok = [i for i in range(16) if score[i] >= score[best] * (1 - 1e-5) and abs(objs[i][1] - d) <= 1e-5 * abs(d)]
        assert ok, (x, d)
        # codes are the nearest entries of x / d, and the scale is fp16(d)
        assert d16 == int(np.array([d], np.float16).view(np.uint16)[0])
        want = _nearest_brute(np.float32(1) / np.float32(d) * x)
        assert np.array_equal(np.concatenate([codes & 15, codes >> 4]), want)
    # every candidate wins somewhere, so a search that drops one fails above
    assert (hist > 0).sum() >= 14, hist


def test_nl4_block_zero_and_tiny():
    d16, codes, d = O.nl4_block(np.zeros(32, np.float32))
    assert d == 0 and d16 == 0 and np.all(codes == 0x88)  # nearest entry to 0 is 1 (index 8)
    x = np.zeros(32, np.float32)
    x[5] = np.float32(9e-16)  # below ggml's 1e-15 group threshold
    assert O.nl4_block(x)[2] == 0
    x[5] = np.float32(1e-15)  # at the threshold: quantized; the fp16 scale underflows to 0
    d16, codes, d = O.nl4_block(x)
    assert d > 0 and d16 == 0 and (codes[5] & 15) in (14, 15)


def test_nl4_rows_source_types_and_layout():
    rng = np.random.default_rng(14)
    rows, cols = 6, 2048
    nb = rows * cols // 32
    # Q8_0 with power-of-two scales: every value is exact in F32, F16 and BF16 as well
    d = (2.0 ** rng.integers(-10, -2, nb)).astype(np.float16)
    q = rng.integers(-127, 128, (nb, 32)).astype(np.int8)
    q8 = np.concatenate([d.view(np.uint8).reshape(nb, 2), q.view(np.uint8)], axis=1)
    x = (d.astype(np.float32)[:, None] * q.astype(np.float32)).reshape(rows, cols)
    ref = O.nl4_quantize_rows(x, O.SRC_F32, rows, cols)
    assert np.array_equal(O.nl4_quantize_rows(q8, O.SRC_Q8_0, rows, cols), ref)
    assert np.array_equal(O.nl4_quantize_rows(x.astype(np.float16), O.SRC_F16, rows, cols), ref)
    bf = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal((bf.astype(np.uint32) << 16).view(np.float32), x)
    assert np.array_equal(O.nl4_quantize_rows(bf, O.SRC_BF16, rows, cols), ref)
    # Q8_0 with arbitrary fp16 scales decodes as fp32(d) * q
    d2 = (rng.random(nb) * 0.01).astype(np.float16)
    q8b = np.concatenate([d2.view(np.uint8).reshape(nb, 2), q.view(np.uint8)], axis=1)
    xb = (d2.astype(np.float32)[:, None] * q.astype(np.float32)).reshape(rows, cols)
    assert np.array_equal(O.nl4_quantize_rows(q8b, O.SRC_Q8_0, rows, cols), O.nl4_quantize_rows(xb, O.SRC_F32, rows, cols))
    # row layout = the one the inference path reads: the NL4 dot of a quantized row
    # against int8 activations equals the float64 dot of its dequantized values
    xa = rng.standard_normal(cols).astype(np.float32)
    xq, xs = O.quant_x(xa)
    act = (xq.astype(np.float64).reshape(-1, 32) * xs.astype(np.float64)[:, None]).reshape(-1)
    deq = O.nl4_dequant_rows(ref, cols).astype(np.float64)
    for r in range(rows):
        got = O.dot_nl4(ref[r], cols, xq, xs)
        assert abs(got - deq[r] @ act) <= 1e-4 * np.abs(deq[r] * act).sum()
    # 4-bit error level of the non-uniform codebook on Gaussian rows
    g = rng.standard_normal((64, cols)).astype(np.float32)
    e = np.linalg.norm(O.nl4_dequant_rows(O.nl4_quantize_rows(g, O.SRC_F32, 64, cols), cols) - g) / np.linalg.norm(g)
    assert 0.05 < e < 0.12, e


def test_convert_expert_row_placement():
    rng = np.random.default_rng(15)
    e = 1  # the oracle reads only expert e's slice, so two experts' worth of source suffice
    n_gu, n_dn = 2 * 512 * 2048 // 32, 2 * 2048 * 512 // 32

    def q8(n):
        d = (rng.random(n) * 0.02).astype(np.float16)
        return np.concatenate([d.view(np.uint8).reshape(n, 2), rng.integers(0, 256, (n, 32), dtype=np.uint8)], 1)

    gate, up, down = q8(n_gu), q8(n_gu), q8(n_dn)
    blob = O.convert_expert(gate, up, down, O.SRC_Q8_0, e)
    half_gu, half_dn = n_gu // 2, n_dn // 2
    assert np.array_equal(blob[:512 * 1152], O.nl4_quantize_rows(gate[half_gu:], O.SRC_Q8_0, 512, 2048).reshape(-1))
    assert np.array_equal(blob[512 * 1152:1024 * 1152], O.nl4_quantize_rows(up[half_gu:], O.SRC_Q8_0, 512, 2048).reshape(-1))
    assert np.array_equal(blob[1024 * 1152:], O.nl4_quantize_rows(down[half_dn:], O.SRC_Q8_0, 2048, 512).reshape(-1))
