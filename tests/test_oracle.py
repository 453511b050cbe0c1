"""CPU tests that pin the oracle (oracle/fgqa_oracle.c) before it is trusted.

The reference ships no golden vectors or fixtures for this path (its checks are
printed, recomputed from random inputs each run), so the oracle is pinned by:
  * the IEEE-754 definition of round-to-nearest-even for bf16 (exhaustive);
  * a float64 brute-force softmax attention, itself checked against an
    independent numpy float64 restatement;
  * closed forms (one token -> V[0], constant V, zero Q -> mean of V, LSE of
    equal logits = log n) and invariants (tile-size invariance, head
    permutation, decode == last causal prefill row, NaN padding never read);
  * planted mistakes (wrong scale, wrong KV-head mapping, causal off by one,
    transposed V) that the tolerance check must reject.
"""
import math

import numpy as np
import pytest

import oracle
from tests._helpers import assert_close, within_tol

SCALE = 1.0 / math.sqrt(128)


# ----------------------------------------------------------------- bf16
def _rne_by_definition(x32: np.ndarray) -> np.ndarray:
    """bf16 RNE from the definition: pick the nearer of the two bf16 neighbours
    (exact distances in float64), ties to the even mantissa."""
    u = x32.view(np.uint32).astype(np.uint64)
    lo = (u >> 16) & 0xFFFF                       # truncation (toward zero)
    hi = lo + 1                                   # next bf16 away from zero
    flo = (lo.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    fhi = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    xv = x32.astype(np.float64)
    dlo = np.abs(xv - flo)
    dhi = np.abs(fhi - xv)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo & 1) == 1))
    return np.where(pick_hi, hi, lo).astype(np.uint16)


def test_bf16_roundtrip_exhaustive():
    L = oracle.lib()
    bits = np.arange(65536, dtype=np.uint16)
    f = oracle.bf16_to_f32(bits)
    back = oracle.f32_to_bf16(f)
    nan = np.isnan(f)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(oracle.bf16_to_f32(back[nan])))
    # C and numpy conversions agree on every bf16 value
    c_back = np.array([L.fgqa_oracle_f32_to_bf16(float(x)) for x in f[::97]], dtype=np.uint16)
    assert np.array_equal(c_back[~np.isnan(f[::97])], bits[::97][~np.isnan(f[::97])])


def test_bf16_rne_ties_and_random():
    # exact midpoints: 1 + 2^-8 lies between 0x3F80 and 0x3F81 -> even 0x3F80;
    # 1 + 3*2^-8 lies between 0x3F81 and 0x3F82 -> even 0x3F82
    cases = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 1 + 2**-8 + 2**-20,
                      3.3895313892515355e38, 3.4028234663852886e38, 0.0, -0.0,
                      1e-45, np.inf, -np.inf], dtype=np.float32)
    expect = np.array([0x3F80, 0x3F82, 0xBF80, 0x3F81, 0x7F7F, 0x7F80, 0, 0x8000, 0, 0x7F80, 0xFF80],
                      dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(cases), expect)
    L = oracle.lib()
    assert [L.fgqa_oracle_f32_to_bf16(float(x)) for x in cases] == list(expect)
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(1 << 20) * np.exp(rng.uniform(-30, 30, 1 << 20))).astype(np.float32)
    finite = np.isfinite(x) & (np.abs(x) < 3.38e38)
    x = x[finite]
    ref = _rne_by_definition(x)
    assert np.array_equal(oracle.f32_to_bf16(x), ref)
    out = np.empty(x.size, dtype=np.uint16)
    L.fgqa_oracle_f32_to_bf16_array(x.ctypes.data_as(oracle.oracle._f32p), out.ctypes.data_as(oracle.oracle._u16p),
                                    x.size)
    assert np.array_equal(out, ref)


# ----------------------------------------------------------------- f64 brute force
def _attention_numpy_f64(q, k, v, scale, causal, seqlens=None, q_offset=0):
    """Independent float64 restatement (BSHD) used to pin the C brute force."""
    qf = oracle.bf16_to_f32(q).astype(np.float64)
    kf = oracle.bf16_to_f32(k).astype(np.float64)
    vf = oracle.bf16_to_f32(v).astype(np.float64)
    B, Sq, Hq, D = qf.shape
    _, Skv, Hkv, _ = kf.shape
    G = Hq // Hkv
    o = np.zeros((B, Sq, Hq, D))
    lse = np.full((B, Hq, Sq), -np.inf)
    for b in range(B):
        n = Skv if seqlens is None else int(seqlens[b])
        for h in range(Hq):
            s = qf[b, :, h, :] @ kf[b, :n, h // G, :].T * scale
            if causal:
                ii = np.arange(Sq)[:, None] + q_offset
                jj = np.arange(n)[None, :]
                s = np.where(jj <= ii, s, -np.inf)
            for i in range(Sq):
                row = s[i]
                if n == 0 or np.all(np.isneginf(row)):
                    continue
                m = row.max()
                e = np.exp(row - m)
                o[b, i, h] = (e / e.sum()) @ vf[b, :n, h // G, :]
                lse[b, h, i] = math.log(e.sum()) + m
    return o, lse


@pytest.mark.parametrize("causal,sq,skv,hq,hkv", [(True, 17, 17, 4, 2), (False, 5, 23, 6, 3), (True, 9, 30, 2, 1)])
def test_f64_bruteforce_matches_numpy(causal, sq, skv, hq, hkv):
    q = oracle.normal_bf16(11, (2, sq, hq, 16))
    k = oracle.normal_bf16(11, (2, skv, hkv, 16), stream=1)
    v = oracle.normal_bf16(11, (2, skv, hkv, 16), stream=2)
    o, lse = oracle.attention_f64(q, k, v, 0.25, causal=causal, causal_offset=3)
    on, ln = _attention_numpy_f64(q, k, v, 0.25, causal, q_offset=3)
    assert np.allclose(o, on, rtol=0, atol=1e-12)
    assert np.allclose(lse, ln, rtol=0, atol=1e-12)
    sl = np.array([skv, 3], dtype=np.int32)
    o, lse = oracle.attention_f64(q, k, v, 0.25, causal=False, seqlens=sl)
    on, ln = _attention_numpy_f64(q, k, v, 0.25, False, seqlens=sl)
    assert np.allclose(o, on, rtol=0, atol=1e-12) and np.allclose(lse, ln, rtol=0, atol=1e-12)


def test_f64_closed_forms():
    # one key -> output is V[0]; equal logits over n keys -> lse = log n + s
    q = np.zeros((1, 1, 2, 8), np.uint16)
    k = oracle.normal_bf16(1, (1, 5, 1, 8))
    v = oracle.normal_bf16(1, (1, 5, 1, 8), stream=2)
    o, lse = oracle.attention_f64(q, k, v, 1.0)
    vf = oracle.bf16_to_f32(v).astype(np.float64)
    assert np.allclose(o[0, 0, 0], vf[0, :, 0].mean(0), atol=1e-14)
    assert np.allclose(lse, math.log(5), atol=1e-14)
    o, _ = oracle.attention_f64(q, k[:, :1], v[:, :1], 1.0)
    assert np.array_equal(o[0, 0, 1], vf[0, 0, 0])


# ----------------------------------------------------------------- decode oracle
def _assert_bf16_rounding_only(out, exact):
    """|out - exact| within one bf16 ulp of |exact| (2^-8 relative) plus the fp32
    accumulation and bf16-P error, which stay below 2e-3 absolute at these sizes."""
    err = np.abs(np.asarray(out, np.float64) - exact)
    bound = np.abs(exact) * 2.0**-8 + 2e-3
    assert np.all(err <= bound), f"worst excess {np.max(err - bound):.3e}"


def _decode_inputs(seed, B, Hq, Hkv, S, D=128):
    q = oracle.normal_bf16(seed, (B, Hq, D))
    k = oracle.normal_bf16(seed, (B, S, Hkv, D), stream=1)
    v = oracle.normal_bf16(seed, (B, S, Hkv, D), stream=2)
    return q, k, v


def _decode_f64(q, k, v, scale, seqlens=None):
    o, lse = oracle.attention_f64(q[:, None], k, v, scale, seqlens=seqlens)
    return o[:, 0], lse[:, :, 0]


@pytest.mark.parametrize("B,Hq,Hkv,S", [(2, 16, 2, 512), (1, 16, 1, 300), (3, 4, 4, 129), (2, 8, 2, 1000)])
def test_decode_oracle_vs_f64(B, Hq, Hkv, S):
    q, k, v = _decode_inputs(3, B, Hq, Hkv, S)
    o, lse = oracle.decode(q, k, v, SCALE)
    of, lf = _decode_f64(q, k, v, SCALE)
    assert_close(oracle.bf16_to_f32(o), of, "decode oracle vs f64")
    _assert_bf16_rounding_only(oracle.bf16_to_f32(o), of)
    assert np.max(np.abs(lse - lf)) < 1e-4


def test_decode_oracle_ragged_and_nan_padding():
    B, Hq, Hkv, S = 6, 8, 2, 300
    q, k, v = _decode_inputs(5, B, Hq, Hkv, S)
    sl = np.array([0, 1, 127, 128, 129, 300], dtype=np.int32)
    o, lse = oracle.decode(q, k, v, SCALE, seqlens=sl)
    of, lf = _decode_f64(q, k, v, SCALE, seqlens=sl)
    assert_close(oracle.bf16_to_f32(o), of, "ragged decode oracle vs f64")
    assert np.all(oracle.bf16_to_f32(o[0]) == 0) and np.all(np.isneginf(lse[0]))
    # padding past each length is never read: NaN there changes nothing
    kn, vn = k.copy(), v.copy()
    for b, n in enumerate(sl):
        kn[b, n:] = 0x7FC0
        vn[b, n:] = 0x7FC0
    o2, lse2 = oracle.decode(q, kn, vn, SCALE, seqlens=sl)
    assert np.array_equal(o, o2) and np.array_equal(lse, lse2)


def test_decode_oracle_known_answers():
    B, Hq, Hkv, S = 2, 8, 2, 257
    q, k, v = _decode_inputs(9, B, Hq, Hkv, S)
    # one token: P = bf16(exp(0)) = 1, l = 1 -> O = V[0] bit-exactly
    o, lse = oracle.decode(q, k[:, :1], v[:, :1], SCALE)
    G = Hq // Hkv
    for h in range(Hq):
        assert np.array_equal(o[:, h], v[:, 0, h // G])
    # Q = 0: every logit is 0 -> O = mean of V over tokens, lse = log S
    qz = np.zeros_like(q)
    o, lse = oracle.decode(qz, k, v, SCALE)
    vm = oracle.bf16_to_f32(v).astype(np.float64).mean(axis=1)  # [B, Hkv, D]
    assert_close(oracle.bf16_to_f32(o), np.repeat(vm, G, axis=1), "Q=0 -> mean(V)", max_abs=4e-3)
    assert np.allclose(lse, math.log(S), atol=1e-5)
    # constant V = c: O = c * sum(bf16 P) / sum(P), within bf16 rounding of P
    c = oracle.f32_to_bf16(np.float32(0.75))
    vc = np.full_like(v, c)
    o, _ = oracle.decode(q, k, vc, SCALE)
    assert np.all(np.abs(oracle.bf16_to_f32(o) - 0.75) <= 0.75 * 2**-7)


def test_decode_oracle_fp32_p_variant():
    """p_bf16=False restates the torch tiled decode reference
    (test_decode_flash_gqa_kernel.py:26-79): the same online softmax with P
    kept in fp32.  It sits closer to the float64 answer than the bf16-P path,
    and with constant V it returns that constant to output rounding."""
    B, Hq, Hkv, S = 2, 16, 2, 1000
    q, k, v = _decode_inputs(17, B, Hq, Hkv, S)
    of, lf = _decode_f64(q, k, v, SCALE)
    o32, l32 = oracle.decode(q, k, v, SCALE, p_bf16=False)
    o16, _ = oracle.decode(q, k, v, SCALE, p_bf16=True)
    e32 = np.abs(oracle.bf16_to_f32(o32) - of)
    e16 = np.abs(oracle.bf16_to_f32(o16) - of)
    _assert_bf16_rounding_only(oracle.bf16_to_f32(o32), of)
    assert e32.mean() < 0.75 * e16.mean(), (e32.mean(), e16.mean())
    assert np.max(np.abs(l32 - lf)) < 1e-4
    c = oracle.f32_to_bf16(np.float32(0.75))
    o, _ = oracle.decode(q, k, np.full_like(v, c), SCALE, p_bf16=False)
    assert np.all(np.abs(oracle.bf16_to_f32(o) - 0.75) <= 0.75 * 2**-9)


def test_decode_oracle_invariants():
    B, Hq, Hkv, S = 2, 16, 2, 700
    q, k, v = _decode_inputs(13, B, Hq, Hkv, S)
    o128, _ = oracle.decode(q, k, v, SCALE, tile=128)
    # flash tile length changes only rounding
    for tile in (37, 512, 4096):
        o_t, _ = oracle.decode(q, k, v, SCALE, tile=tile)
        assert_close(oracle.bf16_to_f32(o_t), oracle.bf16_to_f32(o128), f"tile {tile}", max_abs=8e-3)
    # permuting query heads inside a group permutes the output exactly
    perm = np.concatenate([np.random.default_rng(0).permutation(8), 8 + np.random.default_rng(1).permutation(8)])
    o_p, _ = oracle.decode(q[:, perm], k, v, SCALE)
    assert np.array_equal(o_p, o128[:, perm])
    # decode == last row of a causal prefill over the same keys
    qp = np.zeros((B, S, Hq, 128), np.uint16)
    qp[:, S - 1] = q
    op, lp = oracle.prefill(qp[:, S - 8:], k, v, SCALE, causal=True, q_offset=S - 8)
    assert_close(oracle.bf16_to_f32(op[:, -1]), oracle.bf16_to_f32(o128), "decode vs prefill last row", max_abs=8e-3)


# ----------------------------------------------------------------- prefill oracle
def _prefill_inputs(seed, B, Sq, Skv, Hq, Hkv, sigma=1.0, D=128):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, D), sigma)
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, D), sigma, stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, D), sigma, stream=2)
    return q, k, v


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 256, 256, 4, 1, True), (2, 64, 64, 4, 2, False), (1, 100, 160, 2, 2, True), (1, 160, 100, 3, 1, True)])
def test_prefill_oracle_vs_f64(B, Sq, Skv, Hq, Hkv, causal):
    q, k, v = _prefill_inputs(21, B, Sq, Skv, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=causal)
    of, lf = oracle.attention_f64(q, k, v, SCALE, causal=causal)
    assert_close(oracle.bf16_to_f32(o), of, "prefill oracle vs f64")
    _assert_bf16_rounding_only(oracle.bf16_to_f32(o), of)
    assert np.max(np.abs(lse - lf)) < 1e-4


def test_prefill_oracle_layouts_rows_and_closed_forms():
    B, S, Hq, Hkv = 2, 96, 4, 2
    q, k, v = _prefill_inputs(23, B, S, S, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    # BHSD layout gives the same numbers
    ob, lb = oracle.prefill(q.transpose(0, 2, 1, 3), k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3), SCALE,
                            causal=True, layout="bhsd")
    assert np.array_equal(ob.transpose(0, 2, 1, 3), o) and np.array_equal(lb, lse)
    # a slice of rows with q_offset equals the same rows of the full run
    os_, ls_ = oracle.prefill(q[:, 40:70], k, v, SCALE, causal=True, q_offset=40)
    assert np.array_equal(os_, o[:, 40:70]) and np.array_equal(ls_, lse[:, :, 40:70])
    # causal row 0 sees only key 0: O = V[0] exactly, lse = q0.k0*scale
    G = Hq // Hkv
    for h in range(Hq):
        assert np.array_equal(o[:, 0, h], v[:, 0, h // G])
    qk0 = (oracle.bf16_to_f32(q[:, 0]).astype(np.float64) *
           np.repeat(oracle.bf16_to_f32(k[:, 0]).astype(np.float64), G, axis=1)).sum(-1) * SCALE
    assert np.allclose(lse[:, :, 0], qk0, atol=1e-5)


def test_prefill_oracle_empty_kv():
    q, k, v = _prefill_inputs(1, 1, 4, 0, 2, 1)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    assert np.all(o == 0) and np.all(np.isneginf(lse))


# ----------------------------------------------------------------- planted mistakes
def test_planted_mistakes_are_caught():
    """Each plausible slip must fail the parity bar against the f64 answer."""
    B, Hq, Hkv, S = 2, 16, 2, 512
    q, k, v = _decode_inputs(31, B, Hq, Hkv, S)
    of, _ = _decode_f64(q, k, v, SCALE)
    good, _ = oracle.decode(q, k, v, SCALE)
    assert within_tol(oracle.bf16_to_f32(good), of)
    # dropped/wrong scale
    bad, _ = oracle.decode(q, k, v, SCALE * 1.5)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    # query head h served by KV head h % Hkv instead of h // G: place q[h] at
    # slot p(h) = (h % Hkv) * G + h // Hkv, whose KV head is h % Hkv
    G = Hq // Hkv
    p_of_h = np.array([(h % Hkv) * G + h // Hkv for h in range(Hq)])
    qslot = np.empty_like(q)
    qslot[:, p_of_h] = q
    bad, _ = oracle.decode(qslot, k, v, SCALE)
    assert not within_tol(oracle.bf16_to_f32(bad)[:, p_of_h], of)
    # V read with tokens and head-dim transposed (first 128 tokens)
    vt = v.copy()
    vt[:, :128, :, :] = v[:, :128, :, :].transpose(0, 3, 2, 1)
    bad, _ = oracle.decode(q, k, vt, SCALE)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    # causal mask off by one in prefill
    qp, kp, vp = _prefill_inputs(33, 1, 64, 64, 2, 1)
    pf, _ = oracle.attention_f64(qp, kp, vp, SCALE, causal=True)
    bad, _ = oracle.prefill(qp, kp, vp, SCALE, causal=True, q_offset=1)
    assert not within_tol(oracle.bf16_to_f32(bad), pf)
    good, _ = oracle.prefill(qp, kp, vp, SCALE, causal=True)
    assert within_tol(oracle.bf16_to_f32(good), pf)
    _assert_bf16_rounding_only(oracle.bf16_to_f32(good), pf)


# ----------------------------------------------------------------- backward oracle
from tests._helpers import assert_grad_close, grad_within_tol  # noqa: E402

# Oracle vs the exact (float64) gradient: the reference's algorithm rounds P
# and dS to bf16 (flash_gqa_backward_kernel.py:263,285), which alone moves
# gradients of the earliest keys by up to ~1.8e-2 relative at these sizes, so
# this pin uses 3e-2 / 3e-3; the GPU is held to 2e-2 / 2e-3 against the oracle.
ORACLE_GRAD_REL = 3e-2
ORACLE_GRAD_MEAN = 3e-3


def _bwd_inputs(seed, B, Sq, Skv, Hq, Hkv, D=128, sigma=1.0):
    q, k, v = _prefill_inputs(seed, B, Sq, Skv, Hq, Hkv, D=D, sigma=sigma)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, D), 1.0, stream=3)
    return q, k, v, do


def _loss_numpy_f64(qf, kf, vf, wf, scale, causal):
    """sum(O * W) for float64 softmax attention over BSHD arrays (numpy only)."""
    B, Sq, Hq, D = qf.shape
    Skv, Hkv = kf.shape[1], kf.shape[2]
    G = Hq // Hkv
    tot = 0.0
    for b in range(B):
        for h in range(Hq):
            s = qf[b, :, h] @ kf[b, :, h // G].T * scale
            if causal:
                ii, jj = np.meshgrid(np.arange(Sq), np.arange(Skv), indexing="ij")
                s = np.where(jj <= ii, s, -np.inf)
            for i in range(Sq):
                if np.all(np.isneginf(s[i])):
                    continue
                e = np.exp(s[i] - s[i].max())
                tot += float(((e / e.sum()) @ vf[b, :, h // G]) @ wf[b, i, h])
    return tot


@pytest.mark.parametrize("causal,sq,skv", [(True, 5, 7), (False, 5, 7), (True, 7, 4)])
def test_backward_f64_matches_finite_differences(causal, sq, skv):
    """The float64 gradient equals central differences of an independent numpy forward."""
    B, Hq, Hkv, D = 2, 4, 2, 8
    q, k, v, do = _bwd_inputs(41, B, sq, skv, Hq, Hkv, D=D)
    dq, dk, dv = oracle.attention_backward_f64(q, k, v, do, 0.3, causal=causal)
    f = [oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v, do)]
    eps = 1e-5
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        base = f[which]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            old = base[idx]
            base[idx] = old + eps
            lp = _loss_numpy_f64(f[0], f[1], f[2], f[3], 0.3, causal)
            base[idx] = old - eps
            lm = _loss_numpy_f64(f[0], f[1], f[2], f[3], 0.3, causal)
            base[idx] = old
            num[idx] = (lp - lm) / (2 * eps)
        assert np.allclose(grad, num, rtol=1e-6, atol=1e-7), (which, np.abs(grad - num).max())


def test_backward_f64_invariants_and_torch_form():
    """Exact-gradient invariants: sum_j dK_j = 0 (softmax ignores a common shift
    of the keys), sum_j dV_j = sum of dO over the group's rows (rows of P sum to
    1).  With O given, delta = sum O*dO as in the torch reference."""
    B, S, Hq, Hkv = 2, 40, 4, 2
    q, k, v, do = _bwd_inputs(43, B, S, S, Hq, Hkv, D=16)
    dq, dk, dv = oracle.attention_backward_f64(q, k, v, do, 0.25, causal=True)
    assert np.abs(dk.sum(1)).max() < 1e-12
    G = Hq // Hkv
    dosum = oracle.bf16_to_f32(do).astype(np.float64).reshape(B, S, Hkv, G, 16).sum(axis=(1, 3))
    assert np.abs(dv.sum(1) - dosum).max() < 1e-12
    # O from the exact forward: the torch-form delta equals the exact one
    of, _ = oracle.attention_f64(q, k, v, 0.25, causal=True)
    o_exact = oracle.f32_to_bf16(of.astype(np.float32))
    dq2, dk2, dv2 = oracle.attention_backward_f64(q, k, v, do, 0.25, causal=True, o=o_exact)
    assert np.array_equal(dv2, dv)
    assert np.abs(dq2 - dq).max() < 2e-2 and np.abs(dq2 - dq).max() > 0


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [
    (1, 192, 192, 16, 1, True), (2, 100, 100, 4, 2, False), (1, 70, 130, 2, 2, True), (1, 130, 70, 6, 3, True)])
def test_backward_oracle_vs_f64(B, Sq, Skv, Hq, Hkv, causal):
    q, k, v, do = _bwd_inputs(45, B, Sq, Skv, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=causal)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=causal)
    eq, ek, ev = oracle.attention_backward_f64(q, k, v, do, SCALE, causal=causal, o=o)
    for name, got, ref in (("dq", dq, eq), ("dk", dk, ek), ("dv", dv, ev)):
        rounded = oracle.bf16_to_f32(oracle.f32_to_bf16(got))
        assert_grad_close(rounded, ref, f"backward oracle {name} vs f64", ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)


def test_backward_oracle_known_answers_and_slices():
    # one key: P = 1, dP_i = dO_i.v_0 = delta_i (O = V[0] exactly), so dS = 0:
    # dQ = dK = 0 exactly and dV_0 = sum of dO over the group's rows
    B, S, Hq, Hkv = 2, 9, 4, 2
    q, k, v, do = _bwd_inputs(47, B, S, 1, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=False)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=False)
    assert np.all(dq == 0) and np.all(dk == 0)
    dosum = oracle.bf16_to_f32(do).astype(np.float64).reshape(B, S, Hkv, 2, 128).sum(axis=(1, 3))
    assert np.allclose(dv[:, 0], dosum, rtol=1e-5, atol=1e-5)
    # row / key slices reproduce the full run bit for bit; BHSD gives the same numbers
    q, k, v, do = _bwd_inputs(49, 1, 80, 80, 4, 1)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    sq_, sk_, sv_ = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, rows=(30, 55), keys=(10, 20))
    assert np.array_equal(sq_[:, 30:55], dq[:, 30:55]) and np.all(np.isnan(sq_[:, :30]))
    assert np.array_equal(sk_[:, 10:20], dk[:, 10:20]) and np.array_equal(sv_[:, 10:20], dv[:, 10:20])
    t = lambda x: x.transpose(0, 2, 1, 3)  # noqa: E731
    bq, bk, bv = oracle.prefill_backward(t(q), t(k), t(v), t(o), lse, t(do), SCALE, causal=True, layout="bhsd")
    assert np.array_equal(bq, dq) and np.array_equal(bk, dk) and np.array_equal(bv, dv)


def test_backward_oracle_invariants():
    """sum_j dK_j ~ 0 and sum_j dV_j ~ sum dO hold for the bf16-rounding
    restatement up to its rounding (measured ~1e-3 and ~3e-4 relative)."""
    B, S, Hq, Hkv = 2, 256, 8, 2
    q, k, v, do = _bwd_inputs(51, B, S, S, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    sk = dk.astype(np.float64).sum(1)
    assert np.abs(sk).max() < 5e-3 * np.abs(dk).astype(np.float64).sum(1).mean()
    dosum = oracle.bf16_to_f32(do).astype(np.float64).reshape(B, S, Hkv, Hq // Hkv, 128).sum(axis=(1, 3))
    assert np.abs(dv.astype(np.float64).sum(1) - dosum).max() < 2e-3 * np.abs(dosum).max()


def test_backward_planted_mistakes_are_caught():
    """Each plausible slip in the backward must fail the bar against f64."""
    B, S, Hq, Hkv = 1, 160, 8, 2
    q, k, v, do = _bwd_inputs(53, B, S, S, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    ref = oracle.attention_backward_f64(q, k, v, do, SCALE, causal=True, o=o)

    def ok(grads):
        return all(grad_within_tol(oracle.bf16_to_f32(oracle.f32_to_bf16(g)), r, ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)
                   for g, r in zip(grads, ref))

    assert ok(oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True))
    # delta dropped (O read as zeros)
    assert not ok(oracle.prefill_backward(q, k, v, np.zeros_like(o), lse, do, SCALE, causal=True))
    # scale slip on dS / the logits
    assert not ok(oracle.prefill_backward(q, k, v, o, lse, do, SCALE * 1.1, causal=True))
    # LSE taken in log2 units
    assert not ok(oracle.prefill_backward(q, k, v, o, lse * np.float32(1.4426950408889634), do, SCALE, causal=True))
    # K and V exchanged
    assert not ok(oracle.prefill_backward(q, v, k, o, lse, do, SCALE, causal=True))
    # causal mask dropped
    assert not ok(oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=False))
    # query heads mapped to KV head h % Hkv instead of h // G
    G = Hq // Hkv
    perm = np.array([(h % Hkv) * G + h // Hkv for h in range(Hq)])
    qs, os_, ds = (np.empty_like(x) for x in (q, o, do))
    qs[:, :, perm], os_[:, :, perm], ds[:, :, perm] = q, o, do
    ls = np.empty_like(lse)
    ls[:, perm] = lse
    gq, gk, gv = oracle.prefill_backward(qs, k, v, os_, ls, ds, SCALE, causal=True)
    assert not ok((gq[:, :, perm], gk, gv))



# ----------------------------------------------------------------- paged / fp8 decode oracle
from tests._helpers import fp8_quantize, make_paged  # noqa: E402


def test_fp8_e4m3_decoding_matches_torch():
    """fgqa_oracle_fp8e4m3_to_f32 on all 256 codes equals torch.float8_e4m3fn."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    ours = oracle.fp8e4m3_to_f32(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert np.array_equal(np.signbit(ours[~nan]), np.signbit(theirs[~nan]))
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9


@pytest.mark.parametrize("page_size", [1, 16, 64])
def test_paged_oracle_bit_identical_to_contiguous(page_size):
    """bf16 pages in random order, scales 1: the same bits as the contiguous decode oracle."""
    rng = np.random.default_rng(page_size)
    B, Hq, Hkv, S = 3, 8, 2, 300
    q, k, v = _decode_inputs(61, B, Hq, Hkv, S)
    lens = np.array([300, 1, 137], dtype=np.int32)
    o_ref, l_ref = oracle.decode(q, k, v, SCALE, seqlens=lens)
    kc, vc, bt = make_paged(k, v, lens, page_size, rng)
    o, lse = oracle.decode_paged(q, kc, vc, bt, lens, SCALE)
    assert np.array_equal(o, o_ref) and np.array_equal(lse, l_ref)
    # a second, different page assignment gives the same bits again
    kc2, vc2, bt2 = make_paged(k, v, lens, page_size, np.random.default_rng(page_size + 100))
    o2, _ = oracle.decode_paged(q, kc2, vc2, bt2, lens, SCALE)
    assert np.array_equal(o2, o_ref)


def test_paged_oracle_fp8_against_f64():
    """fp8 caches: the oracle equals the fp64 attention over the decoded values
    (scores scaled by k_scale, output by v_scale) at the parity bar; wrong
    scales or a wrong page are caught."""
    rng = np.random.default_rng(7)
    B, Hq, Hkv, S = 2, 16, 2, 400
    q = oracle.normal_bf16(63, (B, Hq, 128))
    kf = rng.standard_normal((B, S, Hkv, 128)).astype(np.float32)
    vf = rng.standard_normal((B, S, Hkv, 128)).astype(np.float32)
    ks, vs = float(np.abs(kf).max() / 448), float(np.abs(vf).max() / 448)
    k8, v8 = fp8_quantize(kf, ks), fp8_quantize(vf, vs)
    lens = np.array([400, 233], dtype=np.int32)
    kc, vc, bt = make_paged(k8, v8, lens, 16, rng)
    o, lse = oracle.decode_paged(q, kc, vc, bt, lens, SCALE, k_scale=ks, v_scale=vs)
    # fp64 reference on the decoded values (exact in bf16: e4m3 is a subset)
    kb = oracle.f32_to_bf16(oracle.fp8e4m3_to_f32(k8))
    vb = oracle.f32_to_bf16(oracle.fp8e4m3_to_f32(v8))
    of, lf = oracle.attention_f64(q[:, None], kb, vb, SCALE * ks, seqlens=lens)
    ref = of[:, 0] * vs
    assert_close(oracle.bf16_to_f32(o), ref, "paged fp8 oracle vs f64")
    assert np.max(np.abs(lse - lf[:, :, 0])) < 1e-4
    bad, _ = oracle.decode_paged(q, kc, vc, bt, lens, SCALE, k_scale=ks, v_scale=vs * 1.1)
    assert not within_tol(oracle.bf16_to_f32(bad), ref)
    bad, _ = oracle.decode_paged(q, kc, vc, bt, lens, SCALE, k_scale=ks * 3, v_scale=vs)
    assert not within_tol(oracle.bf16_to_f32(bad), ref)
    # (key order does not matter to decode, so a swapped pair of pages is no
    # mistake; a page pointing at unused cache memory is)
    bt_bad = bt.copy()
    used = set(bt[0, :25].tolist()) | set(bt[1, :15].tolist())
    bt_bad[0, 3] = next(pg for pg in range(kc.shape[0]) if pg not in used)
    bad, _ = oracle.decode_paged(q, kc, vc, bt_bad, lens, SCALE, k_scale=ks, v_scale=vs)
    assert not within_tol(oracle.bf16_to_f32(bad)[0], ref[0])


# ----------------------------------------------------------------- sliding window + sink oracle
def _swa_numpy_f64(q, k, v, scale, window, sink):
    """float64 restatement of test_flash_swa_kernel.py:97-116 (BSHD)."""
    qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
    B, Sq, Hq, D = qf.shape
    Skv, Hkv = kf.shape[1], kf.shape[2]
    G = Hq // Hkv
    o = np.zeros((B, Sq, Hq, D))
    lse = np.zeros((B, Hq, Sq))
    for b in range(B):
        for h in range(Hq):
            s = qf[b, :, h] @ kf[b, :, h // G].T * scale
            ii, jj = np.meshgrid(np.arange(Sq), np.arange(Skv), indexing="ij")
            s = np.where((jj <= ii) & (jj >= ii - (window - 1)), s, -np.inf)
            for i in range(Sq):
                if np.all(np.isneginf(s[i])):
                    lse[b, h, i] = math.log(max(sink[h], 1e-9))
                    continue
                m = s[i].max()
                e = np.exp(s[i] - m)
                den = e.sum() + sink[h] * math.exp(-m)
                o[b, i, h] = (e / den) @ vf[b, :, h // G]
                lse[b, h, i] = math.log(den) + m
    return o, lse


def test_swa_oracle_reduces_to_causal_prefill():
    """A window covering the whole sequence and no sink: the causal prefill oracle, bit for bit."""
    q, k, v = _prefill_inputs(71, 2, 150, 150, 4, 2)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    ow, lw = oracle.prefill_swa(q, k, v, SCALE, window=150)
    assert np.array_equal(o, ow) and np.array_equal(lse, lw)


@pytest.mark.parametrize("window,sq,skv", [(1, 40, 40), (7, 60, 60), (32, 90, 90), (16, 50, 30)])
def test_swa_oracle_vs_numpy_f64(window, sq, skv):
    q, k, v = _prefill_inputs(73 + window, 1, sq, skv, 4, 2, D=32)
    sink = np.array([0.5, 2.0, 1e-6, 30.0], dtype=np.float32)
    o, lse = oracle.prefill_swa(q, k, v, 0.2, window=window, sink=sink)
    of, lf = _swa_numpy_f64(q, k, v, 0.2, window, sink)
    assert_close(oracle.bf16_to_f32(o), of, f"swa window={window}")
    assert np.max(np.abs(lse - lf)) < 1e-4
    if window == 1:
        # closed form: row i sees only key i: O = V[i] / (1 + sink exp(-s_ii))
        qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
        s = np.einsum("bihd,bihd->bih", qf, np.repeat(kf, 2, axis=2)) * 0.2
        ref = vf.repeat(2, axis=2) / (1 + sink[None, None, :, None] * np.exp(-s)[..., None])
        assert_close(oracle.bf16_to_f32(o), ref, "swa window=1 closed form")
    # planted mistakes: window off by one, sink dropped, sink taken as a logit
    bad, _ = oracle.prefill_swa(q, k, v, 0.2, window=window + 1, sink=sink)
    if window < sq:
        assert not within_tol(oracle.bf16_to_f32(bad), of)
    bad, _ = oracle.prefill_swa(q, k, v, 0.2, window=window, sink=None)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    bad, _ = oracle.prefill_swa(q, k, v, 0.2, window=window, sink=np.exp(sink))
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    if sq > skv + window - 1:   # rows past every window: O = 0, lse = log(max(sink, 1e-9))
        r = skv + window - 1
        assert np.all(o[:, r:] == 0)
        assert np.allclose(lse[:, :, r:], np.log(np.maximum(sink, 1e-9))[None, :, None])


# ----------------------------------------------------------------- MLA prefill oracle (Dqk != Dv)
def _mla_inputs(seed, B, Sq, Skv, Hq, Hkv, Dqk, Dv, uniform=False):
    if uniform:   # the reference test's inputs: torch.rand, U[0, 1)
        rng = np.random.default_rng(seed)
        mk = lambda shape: oracle.f32_to_bf16(rng.random(shape, dtype=np.float32))  # noqa: E731
        return mk((B, Sq, Hq, Dqk)), mk((B, Skv, Hkv, Dqk)), mk((B, Skv, Hkv, Dv))
    q = oracle.normal_bf16(seed, (B, Sq, Hq, Dqk))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, Dqk), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, Dv), stream=2)
    return q, k, v


def _mla_numpy_f64(q, k, v, scale, causal):
    """float64 restatement of test_flash_mla_kernel.py:27-95 (BSHD, top-left causal)."""
    qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
    B, Sq, Hq, _ = qf.shape
    Skv, Hkv, Dv = kf.shape[1], kf.shape[2], vf.shape[3]
    G = Hq // Hkv
    o = np.zeros((B, Sq, Hq, Dv))
    lse = np.zeros((B, Hq, Sq))
    ii, jj = np.meshgrid(np.arange(Sq), np.arange(Skv), indexing="ij")
    for b in range(B):
        for h in range(Hq):
            s = qf[b, :, h] @ kf[b, :, h // G].T * scale
            if causal:
                s = np.where(jj <= ii, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            e = np.exp(s - m)
            den = e.sum(axis=1, keepdims=True)
            o[b, :, h] = (e / den) @ vf[b, :, h // G]
            lse[b, h] = np.log(den[:, 0]) + m[:, 0]
    return o, lse


def test_mla_oracle_equals_gqa_oracle_when_dims_match():
    """Dqk = Dv = 128: the MLA entry is the prefill oracle, bit for bit (both layouts)."""
    q, k, v = _prefill_inputs(81, 2, 70, 90, 4, 2)
    for causal in (True, False):
        o, lse = oracle.prefill(q, k, v, SCALE, causal=causal)
        om, lm = oracle.prefill_mla(q, k, v, SCALE, causal=causal)
        assert np.array_equal(o, om) and np.array_equal(lse, lm)
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))  # noqa: E731
    ob, lb = oracle.prefill_mla(t(q), t(k), t(v), SCALE, causal=True, layout="bhsd")
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    assert np.array_equal(t(ob), o) and np.array_equal(lb, lse)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal,uniform", [
    (1, 96, 96, 2, 2, True, False), (1, 64, 80, 4, 2, False, False),
    (2, 70, 50, 2, 1, True, False), (1, 128, 128, 2, 2, True, True)])
def test_mla_oracle_vs_numpy_f64(B, Sq, Skv, Hq, Hkv, causal, uniform):
    Dqk, Dv = 192, 128
    scale = 1.0 / math.sqrt(Dqk)   # the reference launcher's default (flash_mla_kernel.py)
    q, k, v = _mla_inputs(83 + Sq, B, Sq, Skv, Hq, Hkv, Dqk, Dv, uniform)
    o, lse = oracle.prefill_mla(q, k, v, scale, causal=causal)
    assert o.shape == (B, Sq, Hq, Dv)
    of, lf = _mla_numpy_f64(q, k, v, scale, causal)
    assert_close(oracle.bf16_to_f32(o), of, "mla vs f64")
    assert np.max(np.abs(lse - lf)) < 1e-4
    if uniform:
        return   # U[0, 1) inputs give near-uniform softmax rows: the mistakes below barely move O
    # planted mistakes: scores over the first 128 dims only; the 1/sqrt(Dv) scale;
    # V read as the first Dv columns of a Dqk-wide row (K in place of V)
    bad, _ = oracle.prefill_mla(q[..., :128], k[..., :128], v, scale, causal=causal)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    bad, _ = oracle.prefill_mla(q, k, v, 1.0 / math.sqrt(Dv), causal=causal)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    bad, _ = oracle.prefill_mla(q, k, np.ascontiguousarray(k[..., :Dv]), scale, causal=causal)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    if causal and Sq <= Skv:
        bad, _ = oracle.prefill_mla(q, k, v, scale, causal=True, q_offset=1)   # causal off by one
        assert not within_tol(oracle.bf16_to_f32(bad), of)


def test_mla_oracle_closed_forms():
    """Causal row 0 = V[0]; Q = 0 gives O_i = mean(V[0..i]) and lse_i = ln(i + 1)."""
    B, S, Hq, Hkv, Dqk, Dv = 1, 60, 2, 1, 192, 128
    q, k, v = _mla_inputs(85, B, S, S, Hq, Hkv, Dqk, Dv)
    o, _ = oracle.prefill_mla(q, k, v, 0.3, causal=True)
    assert np.array_equal(o[:, 0, 0], v[:, 0, 0]) and np.array_equal(o[:, 0, 1], v[:, 0, 0])
    qz = np.zeros_like(q)
    o, lse = oracle.prefill_mla(qz, k, v, 0.3, causal=True)
    vf = oracle.bf16_to_f32(v).astype(np.float64)[0, :, 0]
    ref = np.cumsum(vf, axis=0) / np.arange(1, S + 1)[:, None]
    for h in range(Hq):
        assert_close(oracle.bf16_to_f32(o)[0, :, h], ref, "mla Q = 0")
        assert np.allclose(lse[0, h], np.log(np.arange(1, S + 1)), atol=1e-5)


# ----------------------------------------------------------------- sparse-index prefill oracle
def _sparse_numpy_f64(q, k, v, idx, scale, causal):
    """float64 restatement of test_flash_sgqa_kernel.py:168-222 (BSHD)."""
    qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
    B, Sq, Hq, D = qf.shape
    Skv, Hkv = kf.shape[1], kf.shape[2]
    G = Hq // Hkv
    o = np.zeros((B, Sq, Hq, D))
    lse = np.full((B, Hq, Sq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            for i in range(Sq):
                j = idx[b, h // G, i].astype(np.int64)
                ok = (j >= 0) & (j < Skv)
                if causal:
                    ok &= j <= i
                if not ok.any():
                    continue
                jj = j[ok]
                s = kf[b, jj, h // G] @ qf[b, i, h] * scale
                m = s.max()
                e = np.exp(s - m)
                o[b, i, h] = (e / e.sum()) @ vf[b, jj, h // G]
                lse[b, h, i] = math.log(e.sum()) + m
    return o, lse


def test_sparse_oracle_dense_lists_equal_the_prefill_oracle():
    """Every row listing keys 0..Skv-1 in order: the causal (and full) prefill oracle, bit for bit."""
    B, S, Hq, Hkv = 1, 80, 4, 2
    q, k, v = _prefill_inputs(91, B, S, S, Hq, Hkv)
    idx = np.broadcast_to(np.arange(S, dtype=np.int32), (B, Hkv, S, S)).copy()
    for causal in (True, False):
        o, lse = oracle.prefill(q, k, v, SCALE, causal=causal)
        os_, ls = oracle.sparse_prefill(q, k, v, idx, SCALE, causal=causal)
        assert np.array_equal(o, os_) and np.array_equal(lse, ls)


@pytest.mark.parametrize("B,S,Hq,Hkv,nsparse,causal", [
    (1, 96, 4, 1, 40, True), (2, 64, 4, 2, 24, True), (1, 70, 2, 2, 33, False)])
def test_sparse_oracle_vs_numpy_f64(B, S, Hq, Hkv, nsparse, causal):
    from tests._helpers import build_sparse_indices
    q, k, v = _prefill_inputs(93 + S, B, S, S, Hq, Hkv, D=64)
    idx = build_sparse_indices(95 + S, B, Hkv, S, S, nsparse, recent=8)
    # edge entries the kernels must skip or keep: out of range, a future key,
    # a key listed twice
    rng = np.random.default_rng(S)
    idx[..., -1] = rng.integers(S, 2 * S, size=idx.shape[:3])
    idx[..., -2] = np.minimum(np.arange(S)[None, None, :] + 3, S - 1)
    idx[..., -3] = idx[..., 0]
    o, lse = oracle.sparse_prefill(q, k, v, idx, 0.15, causal=causal)
    of, lf = _sparse_numpy_f64(q, k, v, idx, 0.15, causal)
    assert_close(oracle.bf16_to_f32(o), of, "sparse vs f64")
    fin = np.isfinite(lf)
    assert np.array_equal(np.isfinite(lse), fin)
    assert np.max(np.abs(lse[fin] - lf[fin])) < 1e-4
    # planted mistakes: causal off by one (future key 3 ahead allowed through a
    # shifted row position); empty (-1) slots gathered as key 0 without being
    # masked; the index list of the query head instead of its kv head;
    # out-of-range entries wrapped into range
    if causal:
        bad, _ = oracle.sparse_prefill(q, k, v, idx, 0.15, causal=True, q_offset=3)
        assert not within_tol(oracle.bf16_to_f32(bad), of)
    wrapped = np.where(idx < 0, 0, idx).astype(np.int32)
    bad, _ = oracle.sparse_prefill(q, k, v, wrapped, 0.15, causal=causal)
    assert not within_tol(oracle.bf16_to_f32(bad), of)
    if Hkv > 1:
        bad, _ = oracle.sparse_prefill(q, k, v, idx[:, ::-1], 0.15, causal=causal)
        assert not within_tol(oracle.bf16_to_f32(bad), of)
    wrapped = np.where(idx >= S, idx - S, idx).astype(np.int32)
    bad, _ = oracle.sparse_prefill(q, k, v, wrapped, 0.15, causal=causal)
    assert not within_tol(oracle.bf16_to_f32(bad), of)


def test_sparse_oracle_closed_forms():
    """One valid entry: O = V[j] exactly, lse = score; no valid entry: O = 0,
    lse = -inf; a key listed twice weighs as its score + ln 2."""
    B, S, Hq, Hkv, n = 1, 40, 2, 1, 8
    q, k, v = _prefill_inputs(97, B, S, S, Hq, Hkv)
    idx = np.full((B, Hkv, S, n), -1, dtype=np.int32)
    idx[0, 0, :, 3] = np.arange(S) // 2          # one causal key per row
    idx[0, 0, 5, :] = -1                          # row 5: nothing valid
    idx[0, 0, 6, 0] = 7                           # row 6: only a future key
    idx[0, 0, 6, 3] = -1
    o, lse = oracle.sparse_prefill(q, k, v, idx, SCALE, causal=True)
    for i in range(S):
        if i in (5, 6):
            assert np.all(o[0, i] == 0) and np.all(np.isneginf(lse[0, :, i]))
        else:
            assert np.array_equal(o[0, i, 0], v[0, i // 2, 0]) and np.array_equal(o[0, i, 1], v[0, i // 2, 0])
    # duplicates: listing key a twice next to key b equals softmax over {a: s_a + ln 2, b: s_b}
    idx2 = np.full((B, Hkv, S, 3), -1, dtype=np.int32)
    idx2[0, 0, :, 0] = 0
    idx2[0, 0, :, 1] = 0
    idx2[0, 0, :, 2] = np.arange(S)
    o2, lse2 = oracle.sparse_prefill(q, k, v, idx2, SCALE, causal=True)
    qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
    for i in range(1, S):
        for h in range(Hq):
            sa = qf[0, i, h] @ kf[0, 0, 0] * SCALE + math.log(2.0)
            sb = qf[0, i, h] @ kf[0, i, 0] * SCALE
            m = max(sa, sb)
            wa, wb = math.exp(sa - m), math.exp(sb - m)
            ref = (wa * vf[0, 0, 0] + wb * vf[0, i, 0]) / (wa + wb)
            assert np.max(np.abs(oracle.bf16_to_f32(o2[0, i, h]) - ref)) < 1e-2
            assert abs(lse2[0, h, i] - (m + math.log(wa + wb))) < 1e-4


# ----------------------------------------------------------------- sliding-window backward oracle
def _loss_swa_numpy_f64(qf, kf, vf, wf, scale, window, sink):
    """sum(O * W) for float64 causal sliding-window attention with a per-head
    sink in the denominator (numpy only, BSHD)."""
    B, Sq, Hq, D = qf.shape
    Skv, Hkv = kf.shape[1], kf.shape[2]
    G = Hq // Hkv
    ii, jj = np.meshgrid(np.arange(Sq), np.arange(Skv), indexing="ij")
    vis = (jj <= ii) & (jj > ii - window)
    tot = 0.0
    for b in range(B):
        for h in range(Hq):
            s = np.where(vis, qf[b, :, h] @ kf[b, :, h // G].T * scale, -np.inf)
            for i in range(Sq):
                if not vis[i].any():
                    continue
                m = s[i].max()
                e = np.exp(s[i] - m)
                den = e.sum() + (0.0 if sink is None else float(sink[h]) * math.exp(-m))
                tot += float(((e / den) @ vf[b, :, h // G]) @ wf[b, i, h])
    return tot


@pytest.mark.parametrize("window,with_sink", [(3, True), (2, False), (10, True)])
def test_swa_backward_f64_matches_finite_differences(window, with_sink):
    B, S, Hq, Hkv, D = 1, 6, 4, 2, 8
    q, k, v, do = _bwd_inputs(61 + window, B, S, S, Hq, Hkv, D=D)
    sink = np.array([0.5, 2.0, 0.1, 4.0], dtype=np.float32) if with_sink else None
    dq, dk, dv = oracle.attention_backward_f64(q, k, v, do, 0.3, causal=True, window=window, sink=sink)
    f = [oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v, do)]
    eps = 1e-5
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        base = f[which]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            old = base[idx]
            base[idx] = old + eps
            lp = _loss_swa_numpy_f64(f[0], f[1], f[2], f[3], 0.3, window, sink)
            base[idx] = old - eps
            lm = _loss_swa_numpy_f64(f[0], f[1], f[2], f[3], 0.3, window, sink)
            base[idx] = old
            num[idx] = (lp - lm) / (2 * eps)
        assert np.allclose(grad, num, rtol=1e-6, atol=1e-7), (which, np.abs(grad - num).max())


def test_swa_backward_oracle_reduces_to_causal_backward():
    """A window covering the sequence: the causal backward oracle, bit for bit."""
    q, k, v, do = _bwd_inputs(63, 1, 90, 90, 4, 2)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    ref = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    got = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=90)
    for a, b in zip(ref, got):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("window,with_sink", [(16, True), (1, True), (40, False)])
def test_swa_backward_oracle_vs_f64(window, with_sink):
    B, S, Hq, Hkv = 1, 120, 8, 2
    q, k, v, do = _bwd_inputs(65 + window, B, S, S, Hq, Hkv)
    sink = (np.linspace(0.2, 3.0, Hq).astype(np.float32)) if with_sink else None
    o, lse = oracle.prefill_swa(q, k, v, SCALE, window, sink)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=window)
    eq, ek, ev = oracle.attention_backward_f64(q, k, v, do, SCALE, causal=True, o=o, window=window, sink=sink)
    for name, got, ref in (("dq", dq, eq), ("dk", dk, ek), ("dv", dv, ev)):
        rounded = oracle.bf16_to_f32(oracle.f32_to_bf16(got))
        assert_grad_close(rounded, ref, f"swa backward oracle {name} vs f64", ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)
    # planted mistakes: window off by one; the LSE of the forward without its sink
    if window > 1:
        bq, bk, bv = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True, window=window + 1)
        assert not grad_within_tol(oracle.bf16_to_f32(oracle.f32_to_bf16(bk)), ek, ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)
    if with_sink:
        _, lse_nosink = oracle.prefill_swa(q, k, v, SCALE, window, None)
        bq, bk, bv = oracle.prefill_backward(q, k, v, o, lse_nosink, do, SCALE, causal=True, window=window)
        assert not grad_within_tol(oracle.bf16_to_f32(oracle.f32_to_bf16(bv)), ev, ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)


# ----------------------------------------------------------------- MLA backward oracle
MLA_SCALE = 1.0 / math.sqrt(192)


def _mla_bwd_inputs(seed, B, Sq, Skv, Hq, Hkv, dqk=192, dv=128):
    q = oracle.normal_bf16(seed, (B, Sq, Hq, dqk))
    k = oracle.normal_bf16(seed, (B, Skv, Hkv, dqk), stream=1)
    v = oracle.normal_bf16(seed, (B, Skv, Hkv, dv), stream=2)
    do = oracle.normal_bf16(seed, (B, Sq, Hq, dv), stream=3)
    return q, k, v, do


@pytest.mark.parametrize("causal,sq,skv", [(True, 5, 6), (False, 4, 7)])
def test_mla_backward_f64_matches_finite_differences(causal, sq, skv):
    """The float64 MLA gradient (Q/K rows of 12, V/O rows of 8) equals central
    differences of an independent numpy forward."""
    B, Hq, Hkv = 1, 4, 2
    q, k, v, do = _mla_bwd_inputs(61, B, sq, skv, Hq, Hkv, dqk=12, dv=8)
    dq, dk, dv = oracle.attention_backward_f64(q, k, v, do, 0.3, causal=causal)
    assert dq.shape[-1] == 12 and dk.shape[-1] == 12 and dv.shape[-1] == 8
    f = [oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v, do)]
    eps = 1e-5
    for which, grad in ((0, dq), (1, dk), (2, dv)):
        base = f[which]
        num = np.zeros_like(base)
        for idx in np.ndindex(base.shape):
            old = base[idx]
            base[idx] = old + eps
            lp = _loss_numpy_f64(f[0], f[1], f[2], f[3], 0.3, causal)
            base[idx] = old - eps
            lm = _loss_numpy_f64(f[0], f[1], f[2], f[3], 0.3, causal)
            base[idx] = old
            num[idx] = (lp - lm) / (2 * eps)
        assert np.allclose(grad, num, rtol=1e-6, atol=1e-7), (which, np.abs(grad - num).max())


def test_mla_backward_oracle_equals_gqa_when_dims_match():
    """The MLA entry point with dqk = dv runs the GQA backward's steps: bit-identical."""
    import ctypes
    B, S, Hq, Hkv = 1, 96, 4, 2
    q, k, v, do = _bwd_inputs(63, B, S, S, Hq, Hkv)
    o, lse = oracle.prefill(q, k, v, SCALE, causal=True)
    ref = oracle.prefill_backward(q, k, v, o, lse, do, SCALE, causal=True)
    outs = [np.full(x.shape, np.nan, dtype=np.float32) for x in ref]
    st = [np.array([S * Hq * 128, Hq * 128, 128], dtype=np.int64), np.array([S * Hkv * 128, Hkv * 128, 128],
                                                                             dtype=np.int64)]
    p16 = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))  # noqa: E731
    pf = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))  # noqa: E731
    pi = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))  # noqa: E731
    rc = oracle.lib().fgqa_oracle_prefill_mla_backward_bf16(
        p16(q), p16(k), p16(v), p16(o), pf(lse), p16(do), SCALE, pf(outs[0]), pf(outs[1]), pf(outs[2]),
        B, S, S, Hq, Hkv, 128, 128, pi(st[0]), pi(st[1]), pi(st[1]), pi(st[0]), pi(st[0]), 1, None, None, 0)
    assert rc == 0
    for a, b in zip(outs, ref):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("B,Sq,Skv,Hq,Hkv,causal", [(1, 128, 128, 4, 4, True), (1, 100, 70, 4, 2, False),
                                                    (2, 64, 96, 2, 1, True)])
def test_mla_backward_oracle_vs_f64(B, Sq, Skv, Hq, Hkv, causal):
    q, k, v, do = _mla_bwd_inputs(65, B, Sq, Skv, Hq, Hkv)
    o, lse = oracle.prefill_mla(q, k, v, MLA_SCALE, causal=causal)
    dq, dk, dv = oracle.prefill_backward(q, k, v, o, lse, do, MLA_SCALE, causal=causal)
    assert dq.shape[-1] == 192 and dk.shape[-1] == 192 and dv.shape[-1] == 128
    eq, ek, ev = oracle.attention_backward_f64(q, k, v, do, MLA_SCALE, causal=causal, o=o)
    for name, got, ref in (("dq", dq, eq), ("dk", dk, ek), ("dv", dv, ev)):
        rounded = oracle.bf16_to_f32(oracle.f32_to_bf16(got))
        assert_grad_close(rounded, ref, f"MLA backward oracle {name} vs f64", ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)


def test_mla_backward_planted_mistakes_are_caught():
    """MLA slips fail the bar against the float64 gradient: scores over the
    first 128 dims only, the 1/sqrt(Dv) scale, dP over half of V's dims."""
    B, S, Hq, Hkv = 1, 128, 4, 2
    q, k, v, do = _mla_bwd_inputs(67, B, S, S, Hq, Hkv)
    o, lse = oracle.prefill_mla(q, k, v, MLA_SCALE, causal=True)
    ref = oracle.attention_backward_f64(q, k, v, do, MLA_SCALE, causal=True, o=o)

    def ok(grads):
        return all(grad_within_tol(oracle.bf16_to_f32(oracle.f32_to_bf16(g)), r, ORACLE_GRAD_REL, ORACLE_GRAD_MEAN)
                   for g, r in zip(grads, ref))

    assert ok(oracle.prefill_backward(q, k, v, o, lse, do, MLA_SCALE, causal=True))
    q128, k128 = q.copy(), k.copy()
    q128[..., 128:] = 0
    k128[..., 128:] = 0
    assert not ok(oracle.prefill_backward(q128, k128, v, o, lse, do, MLA_SCALE, causal=True))
    assert not ok(oracle.prefill_backward(q, k, v, o, lse, do, 1.0 / math.sqrt(128), causal=True))
    vh = v.copy()
    vh[..., 64:] = 0
    assert not ok(oracle.prefill_backward(q, k, vh, o, lse, do, MLA_SCALE, causal=True))
