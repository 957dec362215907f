"""Pin the CPU oracle (oracle/moe_oracle.c) before trusting it as the checker.

Checks come from the reference's own known answers (dequant.rs:808-837,
activation.rs:67-81, train.rs:1151-1184), closed forms over every input a
function can see (all fp16 patterns, all 16 MXFP4 codes x 256 exponents),
hand-built bit patterns for each branch of get_scale_min_k4, brute force on
small inputs, and independent numpy f64 restatements (tests/npref.py).
"""
import math

import numpy as np
import pytest

import npref
import oracle
from moe_rocm import synth as S
from moe_rocm import workloads as W


# ---- fp16 / e8m0 -----------------------------------------------------------

def test_fp16_kat_reference():
    # dequant.rs:808-816
    assert oracle.fp16_to_f32(0x3C00) == 1.0
    assert oracle.fp16_to_f32(0x0000) == 0.0
    assert oracle.fp16_to_f32(0xBC00) == -1.0


def test_fp16_exhaustive_vs_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_e8m0_half_closed_form_all_bytes():
    for e in range(256):
        want = np.float32(math.ldexp(1.0, e - 128))
        assert np.float32(oracle.e8m0_to_f32_half(e)).view(np.uint32) == want.view(np.uint32), e


# ---- MXFP4 -----------------------------------------------------------------

def _all_code_blocks():
    """256 blocks, one per exponent; byte j holds code j (low) and 15-j (high)."""
    blocks = np.zeros((256, 17), dtype=np.uint8)
    blocks[:, 0] = np.arange(256)
    j = np.arange(16)
    blocks[:, 1:] = (j | ((15 - j) << 4)).astype(np.uint8)
    return blocks.reshape(-1)


def test_mxfp4_dequant_closed_form_every_code_and_exponent():
    blocks = _all_code_blocks()
    got = oracle.dequant_mxfp4(blocks, 256 * 32).reshape(256, 32)
    mag = [0, 1, 2, 3, 4, 6, 8, 12]
    for e in range(256):
        for j in range(16):
            for code, pos in ((j, j), (15 - j, j + 16)):
                v = math.ldexp(mag[code & 7], e - 128) * (-1 if code >= 8 else 1)
                want = np.float32(v) if code != 8 else np.float32(-0.0)
                assert got[e, pos].view(np.uint32) == want.view(np.uint32), (e, code)


def test_mxfp4_dequant_matches_numpy_restatement_random():
    blk = S.mxfp4_blocks(S.stream_seed(900, 0, 0, 0), 4096)
    a = oracle.dequant_mxfp4(blk, 4096 * 32)
    b = npref.mxfp4_dequant(blk, 4096 * 32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_mxfp4_matvec_one_hot_is_exact_column():
    out_f, in_f = 64, 256
    w = S.mxfp4_blocks(S.stream_seed(901, 0, 0, 0), out_f * in_f // 32)
    W_ = npref.mxfp4_dequant(w, out_f * in_f).reshape(out_f, in_f)
    for col in (0, 5, 16, 31, 32, 100, 255):
        x = np.zeros(in_f, dtype=np.float32)
        x[col] = 1.0
        y = oracle.mxfp4_matvec(w, x, out_f, in_f)
        assert np.array_equal(y, W_[:, col]), col


def test_mxfp4_matvec_f64_bound_and_threads_identical():
    out_f, in_f = 96, 2880
    w = S.mxfp4_blocks(S.stream_seed(902, 0, 0, 0), out_f * in_f // 32)
    x = S.normal(S.stream_seed(902, 1, 0, 0), in_f)
    W_ = npref.mxfp4_dequant(w, out_f * in_f).reshape(out_f, in_f).astype(np.float64)
    y1 = oracle.mxfp4_matvec(w, x, out_f, in_f, 1)
    y8 = oracle.mxfp4_matvec(w, x, out_f, in_f, 8)
    assert np.array_equal(y1, y8)  # each row is sequential: thread split cannot change bits
    ref = W_ @ x.astype(np.float64)
    bound = in_f * 2 ** -23 * (np.abs(W_) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(y1 - ref) <= bound)


# ---- Q4_K ------------------------------------------------------------------

def _q4k_block(d=1.0, dmin=0.0, scales=None, qs=None):
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = np.array([d], dtype=np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], dtype=np.float16).view(np.uint8)
    if scales is not None:
        b[4:16] = scales
    if qs is not None:
        b[16:144] = qs
    return b


def test_q4k_reference_kat():
    # dequant.rs:818-837: d=1, dmin=0, scales[0..4]=1 -> result[0] == 0
    b = _q4k_block(1.0, 0.0, scales=np.array([1, 1, 1, 1] + [0] * 8, dtype=np.uint8))
    y = oracle.dequant_q4k(b, 256)
    assert y.shape == (256,) and y[0] == 0.0


def test_q4k_identity_scales_give_codes():
    # sc = 1 for all 8 sub-blocks (j<4: q[j]&63; j>=4: q[j+4]&15 | (q[j-4]>>6)<<4)
    scales = np.zeros(12, dtype=np.uint8)
    scales[0:4] = 1
    scales[8:12] = 1  # low nibbles -> sc for j=4..7, high nibbles -> m = 0
    qs = np.arange(128, dtype=np.uint8)
    y = oracle.dequant_q4k(_q4k_block(1.0, 0.0, scales, qs), 256).reshape(8, 32)
    q = qs.reshape(4, 32)
    for sub in range(8):
        want = ((q[sub // 2] >> (4 * (sub % 2))) & 0xF).astype(np.float32)
        assert np.array_equal(y[sub], want), sub


def test_q4k_mins_only():
    # q = 0, dmin = 1, m_j = j+1 (low branch) / high branch values -> y = -m
    scales = np.zeros(12, dtype=np.uint8)
    scales[4:8] = np.arange(1, 5)             # m for j = 0..3
    scales[8:12] = (np.arange(5, 9) << 4)     # m for j = 4..7 (high nibble of q[j+4])
    y = oracle.dequant_q4k(_q4k_block(0.5, 1.0, scales, np.zeros(128, np.uint8)), 256).reshape(8, 32)
    for sub in range(8):
        assert np.all(y[sub] == -float(sub + 1)), sub


def _pack_q4k_scales(sc, m):
    """The packing side of the format (ggml's Q4_K quantizer writes the 8 six-bit
    (scale, min) pairs this way): pairs 0-3 in the low 6 bits of bytes j and j+4; pairs
    4-7 as nibbles of byte j+4, their high 2 bits in the top bits of bytes j-4 (scale)
    and j (min). The inverse of get_scale_min_k4, written from the packing rule."""
    q = np.zeros(12, dtype=np.int64)
    for j in range(8):
        if j < 4:
            q[j] |= sc[j]
            q[j + 4] |= m[j]
        else:
            q[j + 4] = (sc[j] & 0xF) | ((m[j] & 0xF) << 4)
            q[j - 4] |= (sc[j] >> 4) << 6
            q[j] |= (m[j] >> 4) << 6
    return q.astype(np.uint8)


@pytest.mark.parametrize("j", range(8))
def test_get_scale_min_k4_pack_unpack_round_trip(j):
    """Every (scale, min) in 0..63 x 0..63 at position j, with random pairs at the other
    seven positions (so a byte read from the wrong source shows up), packed and unpacked:
    all eight pairs come back. A swapped high-bit source (q[j-4] vs q[j]) fails here."""
    rng = np.random.default_rng(100 + j)
    for s in range(64):
        for mm in range(64):
            sc = rng.integers(0, 64, 8)
            m = rng.integers(0, 64, 8)
            sc[j], m[j] = s, mm
            q = _pack_q4k_scales(sc, m)
            for jj in range(8):
                assert oracle.get_scale_min_k4(jj, q) == (sc[jj], m[jj]), (j, s, mm, jj)


def test_q4k_hand_worked_block_high_bits():
    """A block worked out by hand with pairs 4-7 above 15 (bits 6-7 of bytes 0-7 set):
    scales (1, 2, 3, 4, 37, 20, 63, 16), mins (0, 5, 10, 15, 50, 33, 17, 63), d = 1,
    dmin = 0.5, every quant byte 0x21 (low nibble 1, high nibble 2). Sub-block s takes
    the low nibbles for even s, high for odd: y_s = sc_s * q - 0.5 * m_s."""
    scales = np.array([129, 66, 195, 68, 192, 133, 74, 207, 37, 20, 31, 240], dtype=np.uint8)
    y = oracle.dequant_q4k(_q4k_block(1.0, 0.5, scales, np.full(128, 0x21, np.uint8)), 256).reshape(8, 32)
    want = [1.0, 1.5, -2.0, 0.5, 12.0, 23.5, 54.5, 0.5]
    for s in range(8):
        assert np.all(y[s] == want[s]), (s, y[s][0])


# ---- MXFP4 multi-token matmul (dequant.rs:705-721) ----------------------------------------

def test_mxfp4_matmul_one_hot_rows_are_exact_columns():
    """Token t's input is one-hot at column c_t: row t of the result is column c_t of the
    dequantized matrix, exactly (pins the [T, in] -> [T, out] layout)."""
    out_f, in_f = 48, 320
    w = S.mxfp4_blocks(S.stream_seed(904, 0, 0, 0), out_f * in_f // 32)
    W_ = npref.mxfp4_dequant(w, out_f * in_f).reshape(out_f, in_f)
    cols = [0, 17, 31, 32, 200, 319]
    x = np.zeros((len(cols), in_f), dtype=np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    y = oracle.mxfp4_matmul(w, x, out_f, in_f)
    for t, c in enumerate(cols):
        assert np.array_equal(y[t], W_[:, c]), t


def test_mxfp4_matmul_f64_bound_and_token_independence():
    """Random tokens against an f64 product with the dequantized matrix (sequential fp32
    sums are within in_f * 2^-23 * |W||x|); the result of a token does not depend on the
    other tokens of the batch (the weights are re-read per token, dequant.rs:705-721)."""
    out_f, in_f, T = 64, 2880, 5
    w = S.mxfp4_blocks(S.stream_seed(905, 0, 0, 0), out_f * in_f // 32)
    x = S.normal(S.stream_seed(905, 1, 0, 0), T * in_f).reshape(T, in_f)
    W_ = npref.mxfp4_dequant(w, out_f * in_f).reshape(out_f, in_f).astype(np.float64)
    y = oracle.mxfp4_matmul(w, x, out_f, in_f, 4)
    ref = x.astype(np.float64) @ W_.T
    bound = in_f * 2 ** -23 * (np.abs(x.astype(np.float64)) @ np.abs(W_).T)
    assert np.all(np.abs(y - ref) <= bound)
    y_rev = oracle.mxfp4_matmul(w, x[::-1].copy(), out_f, in_f, 1)[::-1]
    assert np.array_equal(y, y_rev)


def test_q4k_dequant_matches_numpy_restatement_random():
    blk = S.q4k_blocks(S.stream_seed(903, 0, 0, 0), 512)
    a = oracle.dequant_q4k(blk, 512 * 256)
    b = npref.q4k_dequant(blk, 512 * 256)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ---- routing ---------------------------------------------------------------

@pytest.mark.parametrize("E,k", [(32, 4), (128, 8), (300, 10), (8, 8)])
@pytest.mark.parametrize("mode", ["softmax_after", "norm", "raw"])
def test_topk_brute_force(E, k, mode):
    rng = np.random.default_rng(E * 31 + k)
    logits = rng.standard_normal((16, E)).astype(np.float32)
    logits[3, 5] = logits[3, 7] = logits[3].max() + 1  # exact tie: lower index first
    logits[4, : E // 2] = -np.inf                      # masked experts never chosen
    sw, norm = mode == "softmax_after", mode == "norm"
    idx, w = oracle.topk_routing(logits, k, norm, sw)
    ridx, rw = npref.topk(logits, k, norm, sw)
    assert np.array_equal(idx, ridx)
    assert np.allclose(w, rw, rtol=2e-6, atol=1e-7)
    if sw or norm:
        assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
    assert list(idx[3][:2]) == [5, 7]
    assert np.all(idx[4] >= E // 2) or k > E // 2


def test_topk_unnormalised_equals_full_softmax():
    rng = np.random.default_rng(7)
    logits = rng.standard_normal((4, 64)).astype(np.float32)
    idx, w = oracle.topk_routing(logits, 6, False, False)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert np.allclose(w, np.take_along_axis(p, idx.astype(np.int64), 1), rtol=2e-6)


def _prob_rank_f32(row, k):
    """Standard-mode ranking written out as the reference does it (layer.rs:2371-2394): max by
    f32::max (NaN ignored), p = exp(l - max) in f32, the sum in expert order, p / sum, then a
    stable sort in which a NaN compares equal to everything (all-NaN rows keep expert order).
    Only used on rows whose exp values are exact (0, 1, NaN) or far apart, so numpy's float32
    exp and glibc's expf agree."""
    finite = row[~np.isnan(row)]
    m = np.float32(finite.max()) if finite.size else np.float32(-np.inf)
    with np.errstate(invalid="ignore", over="ignore"):
        e = np.exp((row - m).astype(np.float32)).astype(np.float32)
        tot = np.float32(0.0)
        for v in e:
            tot = np.float32(tot + v)
        p = (e / tot).astype(np.float32)
    if np.isnan(p).all():
        order = np.arange(len(row))
    else:
        assert not np.isnan(p).any()
        order = np.argsort(-p.astype(np.float64), kind="stable")
    return order[:k], p


@pytest.mark.parametrize("pattern", ["equal-probability", "underflow", "nan", "inf", "all-neg-inf"])
def test_topk_standard_mode_ranks_probabilities(pattern):
    """Distinct logits whose probabilities are equal tie (lower index first), not ranked by
    logit; NaN probabilities (a NaN logit, a +inf maximum, a row of -inf) give experts 0..k-1
    with NaN weights. Each pattern is checked to differ from ranking by logit."""
    E, k = 40, 2 if pattern == "equal-probability" else 3
    row = (np.random.default_rng(5).random(E) * 0.05).astype(np.float32)
    if pattern == "equal-probability":   # expf(l - max) == 1.0f for all three
        b = np.float32(0.125)
        row[7], row[9], row[2] = b, b - np.spacing(b), b - 2 * np.spacing(b)
    elif pattern == "underflow":         # expf(< -104) == 0: every other probability is 0
        row = np.random.default_rng(6).uniform(-200, -150, E).astype(np.float32)
        row[7] = 0.0
    elif pattern == "nan":
        row[5] = np.nan
    elif pattern == "inf":
        row[5] = np.inf
    else:
        row[:] = -np.inf
    want, p = _prob_rank_f32(row, k)
    by_logit = np.argsort(-row.astype(np.float64), kind="stable")[:k]
    if pattern != "all-neg-inf":
        assert set(want.tolist()) != set(by_logit.tolist())
    for norm in (False, True):
        idx, w = oracle.topk_routing(row[None, :], k, norm, False)
        assert idx[0].tolist() == want.tolist(), (pattern, idx[0], want)
        if pattern in ("nan", "inf", "all-neg-inf"):
            assert idx[0].tolist() == list(range(k)) and np.isnan(w).all()
        else:
            ref = p[want] / (p[want].sum(dtype=np.float32) if norm else np.float32(1.0))
            assert np.allclose(w[0], ref, rtol=1e-6, atol=0.0)


# ---- activations -------------------------------------------------------------

def test_silu_reference_kat():
    # activation.rs:67-81 (up = 1)
    assert abs(oracle.silu_mul(1.0, 1.0) - 0.7311) < 0.01
    assert abs(oracle.silu_mul(-1.0, 1.0) - (-0.2689)) < 0.01
    assert abs(oracle.silu_mul(0.0, 1.0)) < 0.001


def test_swiglu_oai_reference_kat():
    # train.rs:1151-1184: gate=10 (clamped to 7), up=3 -> about 28
    assert abs(oracle.swiglu_oai(10.0, 3.0) - 28.0) < 0.5


@pytest.mark.parametrize("g,u", [(0.3, -0.7), (7.0, 1.0), (9.5, 8.0), (-3.0, -9.0), (-20.0, 2.0),
                                 (2.5, 7.0), (6.99, -6.99), (0.0, 0.0)])
def test_activation_closed_forms(g, u):
    assert oracle.swiglu_oai(g, u) == pytest.approx(npref.swiglu_oai(g, u), rel=2e-6, abs=1e-7)
    assert oracle.silu_mul(g, u) == pytest.approx(npref.silu_mul(g, u), rel=2e-6, abs=1e-7)
    assert oracle.sigmoid(g) == pytest.approx(npref.sigmoid(g), rel=2e-6, abs=1e-7)


# ---- whole layer -------------------------------------------------------------

TINY_MX = W.LayerSpec(101, 0, W.GGML_MXFP4, 256, 192, 8, 2, W.ROUTE_SOFTMAX_AFTER_TOPK,
                      W.ACT_SWIGLU_OAI, True, True)
TINY_Q4 = W.LayerSpec(102, 0, W.GGML_Q4_K, 512, 256, 16, 4, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                      False, False)
TINY_SH = W.LayerSpec(103, 0, W.GGML_Q4_K, 512, 256, 24, 5, W.ROUTE_NORM_TOPK, W.ACT_SILU,
                      False, False, sh_inter=256)


@pytest.mark.parametrize("spec", [TINY_MX, TINY_Q4, TINY_SH], ids=["mxfp4", "q4k", "q4k+shared"])
def test_layer_matches_f64_restatement(spec):
    host = W.host_layer(spec)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(spec, 3)
    y, idx, w, lg = L.forward(x)
    ry, ridx, rw, rlg = npref.moe_forward(host, x)
    assert np.allclose(lg, rlg, rtol=1e-5, atol=1e-5)
    assert np.array_equal(idx, ridx)
    scale = np.abs(ry).max()
    assert np.abs(y - ry).max() <= 1e-5 * scale


def test_layer_linear_in_routing_weights():
    host = W.host_layer(TINY_MX)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(TINY_MX, 1)
    idx = np.array([[1, 6]], dtype=np.uint32)
    w1 = np.array([[0.25, 0.5]], dtype=np.float32)
    w2 = np.array([[0.5, 0.125]], dtype=np.float32)
    ya = L.experts(x, idx, w1)
    yb = L.experts(x, idx, w2)
    yab = L.experts(x, idx, w1 + w2)
    assert np.allclose(yab, ya + yb, rtol=1e-5, atol=1e-5 * np.abs(yab).max())


def test_layer_single_expert_identity():
    host = W.host_layer(TINY_MX)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(TINY_MX, 1)
    for e in (0, 3, 7):
        y = L.experts(x, np.array([[e, e]], dtype=np.uint32), np.array([[1.0, 0.0]], np.float32))
        o = npref.expert_ffn(host, e, x[0].astype(np.float64))
        assert np.abs(y[0] - o).max() <= 1e-5 * np.abs(o).max()


def test_layer_zero_codes_give_bias_only():
    host = W.host_layer(TINY_MX)
    for name in ("gate", "up", "down"):
        blk = host[name].reshape(-1, 17).copy()
        blk[:, 1:] = 0  # all codes 0 -> W = 0
        host[name] = blk.reshape(-1)
    L = oracle.layer_from_host(host)
    x = W.x_tokens(TINY_MX, 1)
    idx = np.array([[2, 5]], dtype=np.uint32)
    w = np.array([[0.75, 0.25]], dtype=np.float32)
    y = L.experts(x, idx, w)
    db = host["down_b"].reshape(8, 256)
    assert np.allclose(y[0], 0.75 * db[2] + 0.25 * db[5], rtol=1e-6, atol=1e-7)


# ---- RMSNorm (ops/norm.rs:32-36) and the residual block (layer.rs:462-473) --------------
def test_rms_norm_reference_kat():
    # norm.rs:44-56: x = [1, 2, 3, 4], w = 1, eps = 1e-6 -> [0.3651, 0.7303, 1.0954, 1.4606] (+-0.01)
    out = oracle.rms_norm(np.array([[1, 2, 3, 4]], np.float32), np.ones(4, np.float32), 1e-6)[0]
    for got, want in zip(out, [0.3651, 0.7303, 1.0954, 1.4606]):
        assert abs(got - want) < 0.01
    # and the closed form: x / sqrt(7.5 + eps)
    assert np.allclose(out, np.arange(1, 5) / math.sqrt(7.5 + 1e-6), rtol=2e-7, atol=0)


@pytest.mark.parametrize("width", [4, 64, 2048, 2880])
def test_rms_norm_matches_f64(width):
    rng = np.random.default_rng(width)
    x = rng.standard_normal((3, width)).astype(np.float32) * np.float32(3.0)
    w = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    out = oracle.rms_norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * w.astype(np.float64)
    # one sequential fp32 sum over `width` squares: relative error well below 1e-5
    assert np.max(np.abs(out - ref) / np.abs(ref).max()) < 1e-5


def test_rms_norm_invariants():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 256).astype(np.float32)
    a = oracle.rms_norm(x, w, 0.0)
    # the weight multiplies last: doubling it doubles the output exactly
    assert np.array_equal(oracle.rms_norm(x, 2 * w, 0.0), 2 * a)
    # scale invariance (eps = 0; powers of two scale every square exactly)
    assert np.array_equal(oracle.rms_norm(4 * x, w, 0.0), a)
    # unit weight: the output's mean square is 1
    u = oracle.rms_norm(x, np.ones(256, np.float32), 0.0)
    assert np.allclose((u.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-6)
    # eps enters under the root: a large eps shrinks the output
    assert np.all(np.abs(oracle.rms_norm(x, w, 100.0)) < np.abs(a) + 1e-7)


@pytest.mark.parametrize("spec", [TINY_Q4, TINY_SH], ids=["q4k", "q4k+shared"])
def test_q4k_layer_thread_split_is_bit_identical(spec):
    """The F32 GEMV rows of the Q4_K path are split over threads; every row keeps its
    sequential sum, so any thread count gives the same bits."""
    L = oracle.layer_from_host(W.host_layer(spec))
    x = W.x_tokens(spec, 2)
    y1 = L.forward(x, n_threads=1)[0]
    for nt in (3, 8):
        assert np.array_equal(L.forward(x, n_threads=nt)[0].view(np.uint32), y1.view(np.uint32)), nt
