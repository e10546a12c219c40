"""Pins of the oracle (CPU): each function is checked against an independent statement of
what the mathematics fixes -- brute force, closed forms, a float64 library matmul -- chosen
so that a plausible slip (dropped bias, swapped gate/up, transposed down, wrong code order,
unstable sort, wrong tie rule) fails one of them.
"""
import numpy as np
import pytest

from kandiga_amd import layout, synth
from oracle import moe_oracle as O


# ---- router ---------------------------------------------------------------------------
def _route_brute(logits, K):
    T, E = logits.shape
    idx = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float64)
    for t in range(T):
        order = sorted(range(E), key=lambda e: (-float(logits[t, e]), e))[:K]
        idx[t] = order
        p = np.exp(logits[t].astype(np.float64) - logits[t].astype(np.float64).max())
        p /= p.sum()                                    # full softmax, then renormalise the K
        w[t] = p[order] / p[order].sum()
    return idx, w


@pytest.mark.parametrize("E,K", [(8, 2), (16, 4), (40, 8), (256, 8), (512, 10)])
def test_route_brute_force(E, K):
    rng = np.random.default_rng(E + K)
    logits = rng.standard_normal((23, E)).astype(np.float32)
    logits[3] = 0.5                                     # all equal: lowest indices win
    logits[4, ::2] = logits[4, 1]                       # many ties
    idx, w = O.route(logits, K)
    bidx, bw = _route_brute(logits, K)
    assert np.array_equal(idx, bidx)
    np.testing.assert_allclose(w, bw, rtol=1e-6)
    assert np.array_equal(idx[3], np.arange(K))
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-6)


def test_route_weights_closed_form():
    # w_i / w_j = exp(l_i - l_j) for selected i, j
    rng = np.random.default_rng(1)
    logits = (rng.standard_normal((9, 64)) * 3).astype(np.float32)
    idx, w = O.route(logits, 6)
    sel = np.take_along_axis(logits, idx, 1).astype(np.float64)
    np.testing.assert_allclose(w[:, 1:] / w[:, :1], np.exp(sel[:, 1:] - sel[:, :1]), rtol=1e-5)
    assert (np.diff(sel, axis=1) <= 0).all()


def test_route_agrees_with_probability_ranking():
    """The reference kernel's fp32 probability ranking (moe_block.metal:419-505) agrees with
    the logit ranking on the seeded inputs; a constructed fp32 probability collision is flagged."""
    shape = synth.SHAPES["h2048-e256-i512-k8-3bit"]
    _x, logits = synth.make_inputs(shape, 4096, 77, zipf=True)
    assert O.route_prob_ties(logits, 8).size == 0
    a, wa = O.route(logits, 8)
    b, wb = O.route_by_probs(logits, 8)
    assert np.array_equal(a, b)
    np.testing.assert_allclose(wa, wb, rtol=2e-6)
    # two distinct logits whose fp32 exp(l - max) round to the same value
    row = np.full((1, 16), -30.0, np.float32)
    row[0, 0] = 0.0
    base = np.float32(-1.0)
    row[0, 5] = base
    row[0, 2] = np.nextafter(base, np.float32(-2.0))   # smaller logit, lower index
    eb = np.exp(np.float32(row[0, 5]))
    ea = np.exp(np.float32(row[0, 2]))
    if eb == ea:  # collision in fp32 exp on this platform
        assert O.route_prob_ties(row, 2).size == 1
        assert O.route(row, 2)[0][0, 1] == 5 and O.route_by_probs(row, 2)[0][0, 1] == 2


# ---- permutation ------------------------------------------------------------------------
@pytest.mark.parametrize("T,K,E", [(1, 8, 256), (7, 3, 5), (300, 8, 16), (64, 10, 512)])
def test_permute_brute_force(T, K, E):
    rng = np.random.default_rng(T * K)
    idx = rng.integers(0, E, size=(T, K)).astype(np.int32)
    if T > 2:
        idx[1] = idx[0]                                # repeated rows
    r = O.permute(idx, E)
    flat = idx.reshape(-1)
    brute = sorted(range(T * K), key=lambda f: (flat[f], f))
    assert np.array_equal(r["perm"], brute)
    assert np.array_equal(r["s_tok"], np.array(brute) // K)
    assert np.array_equal(r["s_k"], np.array(brute) % K)
    assert np.array_equal(r["counts"], np.bincount(flat, minlength=E))
    assert r["offsets"][0] == 0 and r["offsets"][-1] == T * K
    assert np.array_equal(np.diff(r["offsets"]), r["counts"])
    assert np.array_equal(r["unique"], np.unique(flat))
    assert np.array_equal(flat[r["perm"]][r["group_starts"][:-1]], r["unique"])


def test_permute_empty():
    r = O.permute(np.zeros((0, 4), np.int32), 8)
    assert r["perm"].size == 0 and r["unique"].size == 0 and r["counts"].sum() == 0


# ---- combine ----------------------------------------------------------------------------
def test_combine_closed_form_and_linearity():
    rng = np.random.default_rng(2)
    y = rng.standard_normal((5, 4, 33)).astype(np.float32)
    w = rng.random((5, 4)).astype(np.float32)
    out = O.combine(y, w)
    np.testing.assert_allclose(out, np.einsum("tkh,tk->th", y.astype(np.float64), w), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(O.combine(2 * y, w), 2 * out, rtol=1e-6)
    one = np.zeros_like(w)
    one[:, 2] = 1
    assert np.array_equal(O.combine(y, one), y[:, 2])


# ---- fp16 conversion --------------------------------------------------------------------
def test_c_fp16_conversion_matches_numpy():
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 6, 20000),
        [0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 2 ** -14, 6.1e-5,
         1 + 2 ** -11, 1 + 3 * 2 ** -11, np.inf, -np.inf],
    ]).astype(np.float32)
    got = O.round_f16(vals)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))


# ---- expert MLP ---------------------------------------------------------------------------
@pytest.mark.parametrize("bits,scale_dtype", [(3, "f16"), (4, "f16"), (3, "bf16"), (4, "bf16")])
def test_switch_mlp_matches_f64_library_matmul(bits, scale_dtype):
    shape = synth.LayerShape(192, 128, 6, 3, bits)
    layer = synth.make_layer(shape, 13, scale_dtype)
    x, logits = synth.make_inputs(shape, 4, 14)
    idx, _ = O.route(logits, 3)
    y = O.switch_mlp(layer, x, idx, bits, scale_dtype, nthreads=3)
    for t in range(4):
        for k in range(3):
            ref = O.expert_mlp_f64(layer, idx[t, k], x[t], bits, scale_dtype)[0]
            err = O.compare(y[t, k], ref)
            assert err["rel_l2"] < 2e-6, (t, k, err)


def test_switch_mlp_threads_do_not_change_result():
    shape = synth.LayerShape(128, 64, 9, 8, 3)
    layer = synth.make_layer(shape, 15)
    x, logits = synth.make_inputs(shape, 3, 16)
    idx, _ = O.route(logits, 8)
    assert np.array_equal(O.switch_mlp(layer, x, idx, 3, nthreads=1), O.switch_mlp(layer, x, idx, 3, nthreads=8))


def _uniform_expert_layer(H, I, bits, cg, cu, cd, s=0.03125, b=-0.0625):
    """One expert whose gate/up/down codes are constant (cg, cu, cd) with one scale/bias."""
    def proj(rows, cols, c):
        codes = np.full((1, rows, cols), c, np.uint8)
        return (layout.pack_codes(codes, bits), np.full((1, rows, cols // 64), s, np.float16).view(np.uint16),
                np.full((1, rows, cols // 64), b, np.float16).view(np.uint16))
    L = {}
    for name, rows, cols, c in (("gate", I, H, cg), ("up", I, H, cu), ("down", H, I, cd)):
        L[f"{name}_w"], L[f"{name}_s"], L[f"{name}_b"] = proj(rows, cols, c)
    return L


def test_switch_mlp_closed_form_uniform_weights():
    """Constant codes: g = wg*sum(x), u = wu*sum(x), act = silu(g)*u for every row,
    y_h = wd * I * act.  Swapping gate/up or dropping a bias changes the value."""
    H, I, bits = 128, 64, 3
    cg, cu, cd, s, b = 5, 6, 7, 0.03125, -0.0625
    L = _uniform_expert_layer(H, I, bits, cg, cu, cd, s, b)
    x = np.linspace(-1, 1, H).astype(np.float16)[None, :] + np.float16(0.25)
    sx = float(x.astype(np.float64).sum())
    wg, wu, wd = cg * s + b, cu * s + b, cd * s + b
    g, u = wg * sx, wu * sx
    act = g / (1 + np.exp(-g)) * u
    y = O.switch_mlp(L, x, np.zeros((1, 1), np.int32), bits)[0, 0]
    np.testing.assert_allclose(y, wd * I * act, rtol=1e-5)
    swapped = u / (1 + np.exp(-u)) * g
    assert abs(swapped - act) > 1e-2 * abs(act)
    no_bias = (cg * s * sx) / (1 + np.exp(-cg * s * sx)) * (cu * s * sx) * (cd * s) * I
    assert abs(no_bias - wd * I * act) > 1e-2 * abs(wd * I * act)


def test_switch_mlp_zero_weights():
    """Codes 2**(b-1) with bias -2**(b-1)*s dequantize to exactly zero."""
    for bits in (3, 4):
        mid = 2 ** (bits - 1)
        L = _uniform_expert_layer(128, 64, bits, mid, mid, mid, s=0.0625, b=-mid * 0.0625)
        x = np.ones((2, 128), np.float16)
        y = O.switch_mlp(L, x, np.zeros((2, 1), np.int32), bits)
        assert np.array_equal(y, np.zeros_like(y))


def test_expert_mlp_detects_transposed_down():
    shape = synth.LayerShape(128, 64, 2, 1, 4)
    layer = synth.make_layer(shape, 17)
    x, _ = synth.make_inputs(shape, 1, 18)
    g, u, d = O.expert_weights_f64(layer, 1, 4, 128, 64)
    xs = x.astype(np.float64)[0]
    a = O.silu64(g @ xs) * (u @ xs)
    good = O.expert_mlp_f64(layer, 1, x, 4)[0]
    np.testing.assert_allclose(good, d @ a, rtol=1e-12)
    # code order slip: reversing codes within each packed word gives a different result
    bad = layer.copy()
    c = layout.unpack_codes(layer["gate_w"], 4, 128)
    bad["gate_w"] = layout.pack_codes(c.reshape(2, 64, 16, 8)[..., ::-1].reshape(2, 64, 128), 4)
    assert O.compare(O.expert_mlp_f64(bad, 1, x, 4)[0], good)["rel_l2"] > 1e-2


def test_moe_layer_end_to_end_small():
    shape = synth.LayerShape(128, 64, 8, 2, 3)
    layer = synth.make_layer(shape, 19)
    x, logits = synth.make_inputs(shape, 6, 20)
    r = O.moe_layer(layer, x, logits, 2, 3)
    ref = np.zeros((6, 128))
    for t in range(6):
        for k in range(2):
            ref[t] += r["w"][t, k] * O.expert_mlp_f64(layer, r["idx"][t, k], x[t], 3)[0]
    assert O.compare(r["out"], ref)["rel_l2"] < 2e-6


def test_golden_fixture_reproduces():
    """tests/golden/moe_small.npz was written by tests/golden/make_golden.py from the oracle."""
    import os
    from tests.golden.make_golden import CASES, build_case

    data = np.load(os.path.join(os.path.dirname(__file__), "golden", "moe_small.npz"))
    for name in CASES:
        case = build_case(name)
        assert case["layer_sha256"] == str(data[f"{name}.layer_sha256"]), f"{name}: generator drift"
        assert np.array_equal(case["idx"], data[f"{name}.idx"])
        assert np.array_equal(case["perm"], data[f"{name}.perm"])
        np.testing.assert_allclose(case["w"], data[f"{name}.w"], rtol=1e-6)
        np.testing.assert_allclose(case["y"], data[f"{name}.y"], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(case["out"], data[f"{name}.out"], rtol=1e-5, atol=1e-6)


# ---- router: NaN and infinities ------------------------------------------------------------
def test_route_nan_and_inf_ordering():
    """NaN logits rank below every number (-inf included), ties among them to the lower index;
    brute force with an explicit (class, value, index) key."""
    rng = np.random.default_rng(8)
    logits = rng.standard_normal((6, 40)).astype(np.float32)
    logits[0, [3, 7, 11]] = np.nan
    logits[1, :] = np.nan
    logits[1, [5, 9]] = -np.inf
    logits[2, ::2] = -np.inf
    logits[3, [0, 1]] = np.inf
    logits[4, :38] = np.nan
    idx, w = O.route(logits, 8)

    def key(v, e):
        return (1, 0.0, e) if np.isnan(v) else (0, -float(v), e)

    for t in range(logits.shape[0]):
        brute = sorted(range(40), key=lambda e: key(logits[t, e], e))[:8]
        assert list(idx[t]) == brute, t
    assert list(idx[1][:2]) == [5, 9] and list(idx[1][2:]) == [0, 1, 2, 3, 4, 6]
    assert np.isnan(w[1]).all() and np.isnan(w[4]).all()   # a selected NaN makes the renorm NaN
    assert not np.isnan(w[0]).any() and not np.isnan(w[2]).any()


# ---- dequantization with general scale/bias pairs ------------------------------------------
def _general_scale_bias(rng, shape, scale_dtype):
    """Independent random scales and biases (not b = -2**(bits-1)*s), both signs, spanning
    2**-13 .. 2**3 in magnitude, as 16-bit patterns of ``scale_dtype``."""
    mag = np.exp2(rng.uniform(-13, 3, size=shape)) * rng.choice([-1.0, 1.0], size=shape)
    if scale_dtype == "f16":
        return layout.f16_bits(mag.astype(np.float16))
    return layout.f32_to_bf16_bits(mag.astype(np.float32))


@pytest.mark.parametrize("bits,scale_dtype", [(3, "f16"), (4, "f16"), (3, "bf16"), (4, "bf16")])
def test_dequantize_brute_force_general_scales(bits, scale_dtype):
    """Element by element: code of column c read from the packed bytes bit by bit (LSB-first
    bit stream), w = q * s[c // 64] + b[c // 64] with Python floats."""
    rng = np.random.default_rng(bits * 10 + len(scale_dtype))
    rows, cols = 3, 192
    codes = rng.integers(0, 2 ** bits, size=(rows, cols))
    words = layout.pack_codes(codes, bits)
    s = _general_scale_bias(rng, (rows, cols // 64), scale_dtype)
    b = _general_scale_bias(rng, (rows, cols // 64), scale_dtype)
    got = O.dequantize(words, s, b, bits, cols, scale_dtype)
    raw = words.view(np.uint8).reshape(rows, -1)

    def f(u):
        if scale_dtype == "f16":
            return float(np.uint16(u).view(np.float16))
        return float(np.uint32(int(u) << 16).view(np.float32))

    for r in range(rows):
        for c in range(cols):
            q = sum(((int(raw[r, (c * bits + i) // 8]) >> ((c * bits + i) % 8)) & 1) << i for i in range(bits))
            assert q == codes[r, c]
            assert got[r, c] == q * f(s[r, c // 64]) + f(b[r, c // 64]), (r, c)


# ---- dense shared expert ------------------------------------------------------------------
def test_shared_expert_closed_form_constant_weights():
    """Constant gate/up/down matrices a, b, c: every intermediate unit is silu(a*S)*(b*S) with
    S = sum(x), and every output is c * Is * that.  A gate/up swap gives a different value."""
    H, Is = 128, 64
    a, b, c = 0.0625, -0.03125, 0.015625
    layer = {"shared_gate": layout.f16_bits(np.full((Is, H), a, np.float16)),
             "shared_up": layout.f16_bits(np.full((Is, H), b, np.float16)),
             "shared_down": layout.f16_bits(np.full((H, Is), c, np.float16))}
    x = (np.linspace(-1, 2, 3 * H).reshape(3, H)).astype(np.float16)
    S = x.astype(np.float64).sum(axis=1, keepdims=True)
    g, u = a * S, b * S
    want = np.repeat(c * Is * (g / (1 + np.exp(-g))) * u, H, axis=1)
    got = O.shared_expert_f64(layer, x)
    np.testing.assert_allclose(got, want, rtol=1e-12)
    swapped = c * Is * (u / (1 + np.exp(-u))) * g
    assert (np.abs(swapped - want[:, :1]) > 1e-2 * np.abs(want[:, :1])).all()


def test_shared_expert_brute_force_loops():
    """Random non-square matrices (H != Is) against explicit index loops: out[t, h] =
    sum_i down[h, i] * silu(sum_j gate[i, j] x[t, j]) * sum_j up[i, j] x[t, j]."""
    rng = np.random.default_rng(21)
    H, Is, T = 24, 16, 3
    gate = (rng.standard_normal((Is, H)) * 0.3).astype(np.float16)
    up = (rng.standard_normal((Is, H)) * 0.3).astype(np.float16)
    down = (rng.standard_normal((H, Is)) * 0.3).astype(np.float16)
    x = rng.standard_normal((T, H)).astype(np.float16)
    layer = {"shared_gate": layout.f16_bits(gate), "shared_up": layout.f16_bits(up),
             "shared_down": layout.f16_bits(down)}
    got = O.shared_expert_f64(layer, x)
    for t in range(T):
        for h in range(H):
            acc = 0.0
            for i in range(Is):
                gi = sum(float(gate[i, j]) * float(x[t, j]) for j in range(H))
                ui = sum(float(up[i, j]) * float(x[t, j]) for j in range(H))
                acc += float(down[h, i]) * (gi / (1 + np.exp(-gi))) * ui
            assert abs(got[t, h] - acc) <= 1e-12 * max(1.0, abs(acc)), (t, h)


# ---- GELU-tanh gate of the C restatement ----------------------------------------------------
def test_switch_mlp_gelu_tanh_matches_torch_gelu():
    """act == 1 (kandiga_cpu_expert_lg.m:237-245) against an f64 reference whose gate activation
    is torch.nn.functional.gelu(approximate='tanh') on the CPU; SwiGLU must differ."""
    import torch

    shape = synth.LayerShape(192, 128, 5, 2, 3)
    for scale_dtype in ("f16", "bf16"):
        layer = synth.make_layer(shape, 23, scale_dtype)
        x, logits = synth.make_inputs(shape, 3, 24)
        idx, _ = O.route(logits, 2)
        y = O.switch_mlp(layer, x, idx, 3, scale_dtype, act="gelu", nthreads=2)
        y_silu = O.switch_mlp(layer, x, idx, 3, scale_dtype, act="silu")
        for t in range(3):
            for k in range(2):
                g_w, u_w, d_w = O.expert_weights_f64(layer, idx[t, k], 3, 192, 128, scale_dtype)
                xs = x[t].astype(np.float64)
                g = torch.from_numpy(g_w @ xs)
                a = torch.nn.functional.gelu(g, approximate="tanh").numpy() * (u_w @ xs)
                ref = d_w @ a
                assert O.compare(y[t, k], ref)["rel_l2"] < 2e-6, (scale_dtype, t, k)
                assert O.compare(y_silu[t, k], ref)["rel_l2"] > 1e-2


# ---- CPU baseline ---------------------------------------------------------------------------
@pytest.mark.parametrize("bits,scale_dtype", [(3, "bf16"), (4, "bf16"), (3, "f16")])
def test_ref_scalar_baseline_computes_the_same_layer(bits, scale_dtype):
    """The CPU baseline (the reference's scalar loops, one accumulator, default contraction)
    agrees with the checker to fp32 accumulation-order accuracy, single- and multi-threaded."""
    shape = synth.LayerShape(256, 128, 8, 4, bits)
    layer = synth.make_layer(shape, 27, scale_dtype)
    x, logits = synth.make_inputs(shape, 3, 28)
    idx, _ = O.route(logits, 4)
    ref = O.switch_mlp(layer, x, idx, bits, scale_dtype)
    for nt in (1, 4):
        got = O.ref_scalar_switch_mlp(layer, x, idx, bits, scale_dtype, nthreads=nt)
        assert O.compare(got, ref)["rel_l2"] < 1e-5


# ---- the MoE block around the routed experts ----------------------------------------------
def test_qlinear_brute_force():
    """qlinear_f64 against explicit loops over rows, columns and the bit stream."""
    rng = np.random.default_rng(41)
    for bits in (3, 4):
        rows, cols = 5, 128
        codes = rng.integers(0, 2 ** bits, size=(rows, cols))
        w = layout.pack_codes(codes, bits)
        s = layout.f16_bits((rng.random((rows, 2)) * 0.1 + 0.01).astype(np.float16))
        b = layout.f16_bits((rng.standard_normal((rows, 2)) * 0.1).astype(np.float16))
        x = rng.standard_normal((3, cols)).astype(np.float16)
        got = O.qlinear_f64(w, s, b, bits, x)
        for t in range(3):
            for r in range(rows):
                acc = 0.0
                for c in range(cols):
                    wv = codes[r, c] * float(s.view(np.float16)[r, c // 64]) + float(b.view(np.float16)[r, c // 64])
                    acc += wv * float(x[t, c])
                assert abs(got[t, r] - acc) <= 1e-9 * max(1.0, abs(acc))


def test_moe_block_composition_closed_form():
    """Zero router weights make every logit 0 (route: experts 0..K-1, weights 1/K) and a zero
    shared gate makes sigmoid = 1/2: out = residual + mean_k y_k + fp16(shared) / 2.  Dropping
    the residual, the gate or the fp16 rounding of the shared output changes the value."""
    shape = synth.LayerShape(128, 64, 6, 3, 3)
    layer = synth.make_layer(shape, 43)
    blk = synth.make_block(shape, 64, 44, bits=4, scale_dtype="bf16")
    mid = layout.f32_to_bf16_bits(np.float32([0.0]))[0]
    for name in ("blk_router", "blk_sgate"):
        blk[f"{name}_w"][:] = 0          # codes 0 ...
        blk[f"{name}_b"][:] = mid         # ... and zero bias: every weight is 0
    x, _ = synth.make_inputs(shape, 4, 45)
    res = (np.random.default_rng(46).standard_normal((4, 128)) * 3).astype(np.float16)
    r = O.moe_block(layer, blk, x, 3, 3, 4, "f16", "bf16", residual=res)
    assert np.array_equal(r["idx"], np.tile(np.arange(3, dtype=np.int32), (4, 1)))
    np.testing.assert_allclose(r["w"], 1 / 3, rtol=1e-6)
    y = O.switch_mlp(layer, x, r["idx"], 3)
    sh = O.switch_mlp(O.block_shared_layer(blk), x, np.zeros((4, 1), np.int32), 4, "bf16")[:, 0]
    sh16 = O.round_f16(sh).astype(np.float64)
    want = res.astype(np.float64) + y.astype(np.float64).mean(axis=1) + 0.5 * sh16
    np.testing.assert_allclose(r["out"], want, rtol=2e-6, atol=2e-6)
    assert np.abs(sh16 - sh).max() > 0                       # the shared output is rounded
    assert np.abs(r["out"] - (want - res)).max() > 1.0       # the residual is in
    assert np.abs(0.5 * sh16).max() > 1e-2                   # the gated shared term matters


# ---- fp32 / bf16 activations (bakan_cpu_expert_mlp, bakan_cpu_expert_mlp_bf16) --------------
def test_switch_mlp_fp32_path_equals_fp16_path_on_fp16_values():
    """The fp32-activation entry widens nothing: on fp16-representable x it runs the same fp32
    arithmetic as the fp16 entry, bit for bit."""
    shape = synth.LayerShape(128, 64, 6, 3, 3)
    layer = synth.make_layer(shape, 71)
    x, logits = synth.make_inputs(shape, 4, 72)
    idx, _ = O.route(logits, 3)
    a = O.switch_mlp(layer, x, idx, 3)
    b = O.switch_mlp(layer, x.astype(np.float32), idx, 3, exact_x=True)
    assert np.array_equal(a, b)


def test_switch_mlp_fp32_activations_against_f64():
    """General fp32 x (not fp16-representable, several magnitudes) against float64 products of
    the dequantized matrices on the same fp32 values; and the batched dense oracle agrees."""
    shape = synth.LayerShape(128, 64, 6, 3, 4)
    layer = synth.make_layer(shape, 73)
    rng = np.random.default_rng(74)
    x = (rng.standard_normal((3, 128)) * np.array([[1.0], [300.0], [1e-3]])).astype(np.float32)
    assert not np.array_equal(x, x.astype(np.float16).astype(np.float32))
    _, logits = synth.make_inputs(shape, 3, 75)
    idx, w = O.route(logits, 3)
    y = O.switch_mlp(layer, x, idx, 4, exact_x=True)
    for t in range(3):
        for k in range(3):
            ref = O.expert_mlp_f64(layer, idx[t, k], x[t], 4, exact_x=True)[0]
            np.testing.assert_allclose(y[t, k], ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())
    dense = O.moe_out_dense(lambda e: {k: v[e] for k, v in layer.items()}, x, idx, w, 4, 128, 64, exact_x=True)
    np.testing.assert_allclose(O.combine(y, w), dense, rtol=2e-5, atol=2e-5 * np.abs(dense).max())
    # rounding x to fp16 instead moves the result past the bar above: the check can tell them apart
    y16 = O.switch_mlp(layer, x, idx, 4)
    assert np.abs(y16 - y).max() > 2e-5 * np.abs(y).max()
