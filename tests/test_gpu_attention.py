"""Prefill attention on the GPU against the oracle within the FP32 tolerance
(src/kernels/attention/prefill64/tests.rs:36-84, static_shift/tests.rs).

A pure prefill takes the products from power-of-two scaled FP16 pairs by default
(focr_attention_prefill_split); `split_products=False` and every prefill over
generated keys take the FP32 matrix-core products (focr_attention_prefill).
Both are held to the same bound."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import host, max_rel, oracle_threads, to_dev

pytestmark = pytest.mark.gpu

CASES = [(70, 3, 65), (300, 5, 262), (257, 0, 257), (160, 16, 144), (129, 1, 128), (40, 0, 3), (95, 10, 90), (600, 0, 0)]


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def close(got, want):
    # The reference's own FP32 attention tolerance (prefill64/tests.rs:76-81)
    # and the north-star metric max|d| / max|ref| <= 1e-5.
    assert np.all(np.abs(got - want) <= 1e-5 * (1.0 + np.abs(want))), float(np.max(np.abs(got - want)))
    assert max_rel(got, want) <= 1e-5


def run(fh, q, k, v, sinks, L, geometry, options, prefix=None, total=None, generated=None, n_heads=16, n_kv=8):
    prefix = L if prefix is None else prefix
    total = L if total is None else total
    kv = fh.CompactKv(to_dev(k), None if generated is None else to_dev(generated), to_dev(v), prefix, total,
                      n_heads, n_kv, 64)
    out = fh.attention_with(to_dev(q), kv, L, fh.Geometry(*geometry), to_dev(sinks), options)
    return host(out).reshape(L, n_heads, 64)


@pytest.mark.parametrize("L,image_start,image_end", CASES)
@pytest.mark.parametrize("exp", ["fast", "exact"])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_online_prefill(fh, L, image_start, image_end, exp, products):
    q = gen.att_values(L * 16 * 64, 17 + L, 3.0)
    k = gen.att_values(L * 16 * 64, 19 + L, 3.0)
    v = gen.att_values(L * 8 * 64, 23 + L, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    opts = fh.PrefillOptions(exp=fh.ExpMode.FAST if exp == "fast" else fh.ExpMode.EXACT,
                             split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, image_start, image_end), opts)
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, image_start, image_end, sinks, exp_fast=exp == "fast")
    close(got, want)


@pytest.mark.parametrize("L,image_start,image_end", CASES[:4])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_static_prefill(fh, L, image_start, image_end, products):
    q = gen.normalized(L * 16 * 64, 17 + L)
    k = gen.normalized(L * 16 * 64, 19 + L)
    v = gen.values(L * 8 * 64, 23 + L, 3.0)
    sinks = gen.values(16, 29, 2.0)
    opts = fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC, split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, image_start, image_end), opts)
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, image_start, image_end, sinks, static=True)
    close(got, want)


@pytest.mark.parametrize("L,prefix,total,offset,image", [(4, 137, 141, 137, (1, 129)), (9, 128, 137, 128, (1, 128)),
                                                         (33, 100, 133, 100, (1, 90)), (40, 3, 43, 3, (1, 3)),
                                                         (5, 250, 300, 295, (0, 0))])
def test_generated_keys(fh, L, prefix, total, offset, image):
    # prefill64/tests.rs:89-153 (mixed caches)
    q = gen.att_values(L * 16 * 64, 71, 3.0)
    pk = gen.att_values(prefix * 16 * 64, 83, 3.0)
    gk = gen.att_values((total - prefix) * 8 * 64, 37, 3.0)
    v = gen.att_values(total * 8 * 64, 117, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    got = run(fh, q, pk, v, sinks, L, (offset, *image), fh.PrefillOptions(), prefix=prefix, total=total, generated=gk)
    want = oracle.attention_prefill(q, pk, v, L, prefix, total, 16, 8, offset, image[0], image[1], sinks, generated_k=gk)
    close(got, want)


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_config4_full_page(fh, static, products):
    # 6,544 tokens, 16 heads x 64, image prefix 4,096,
    # Q/K/V ~ N(0,1); every output against the oracle's tiles (their
    # lane-vectorized restatement, bitwise the oracle), online softmax with
    # the Fast exp, and the static-shift softmax.
    L, image_end = 6544, 4096
    q = gen.normal(L * 16 * 64, 1.0, 20)
    k = gen.normal(L * 16 * 64, 1.0, 21)
    v = gen.normal(L * 8 * 64, 1.0, 22)
    sinks = gen.uniform(16, -2.0, 2.0, 23)
    if static:  # the static shift needs bounded scores (prefill64/static_shift.rs)
        q = gen.normalized(L * 16 * 64, 24)
        k = gen.normalized(L * 16 * 64, 25)
    opts = fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE,
                             split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, 0, image_end), opts)
    assert np.all(np.isfinite(got))
    oracle.set_threads(oracle_threads())
    want = oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, 0, image_end, sinks, static=static)
    close(got, want)
    # The restatement against the scalar oracle on tiles of every kind:
    # image-only, straddling the image end, causal, last.
    for t0, t1 in ((0, 1), (127, 129), (204, 205)):
        sl = slice(t0 * 32, min(t1 * 32, L))
        ref = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, 0, image_end, sinks, static=static, tiles=(t0, t1))
        assert np.array_equal(want[sl].view(np.uint32), ref[sl].view(np.uint32))


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("exp", ["fast", "exact"])
def test_split_key_ranges_full_compare(fh, static, exp):
    # 3,000 queries: tiles with more than 1,024 visible keys run as several
    # work items whose softmax states are merged; every row against the oracle.
    # Norm-8 heads bound the logits by 8 (prefill64/test_data.rs:14-23), the
    # regime in which a 1e-5 relative bound is meaningful for long rows.
    if static and exp == "exact":
        pytest.skip("the static softmax has one exp")
    oracle.set_threads(8)
    L, image = 3000, (0, 1500)
    q = gen.normalized(L * 16 * 64, 301)
    k = gen.normalized(L * 16 * 64, 302)
    v = gen.att_values(L * 8 * 64, 303, 3.0)
    sinks = gen.att_values(16, 29, 2.0)
    opts = fh.PrefillOptions(exp=fh.ExpMode.FAST if exp == "fast" else fh.ExpMode.EXACT,
                             fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE)
    got = run(fh, q, k, v, sinks, L, (0, *image), opts)
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, *image, sinks, static=static, exp_fast=exp == "fast")
    close(got, want)


def test_config5_prefill_whole(fh):
    # BASELINE config 5's prefill attention: 16,320 rows, image [0, 4096),
    # split key ranges; every output.
    oracle.set_threads(oracle_threads())
    L, image_end = 16320, 4096
    q = gen.normal(L * 16 * 64, 1.0, 40)
    k = gen.normal(L * 16 * 64, 1.0, 41)
    v = gen.normal(L * 8 * 64, 1.0, 42)
    sinks = gen.uniform(16, -2.0, 2.0, 43)
    got = run(fh, q, k, v, sinks, L, (0, 0, image_end), fh.PrefillOptions())
    assert np.all(np.isfinite(got))
    close(got, oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, 0, image_end, sinks))


def test_more_queries_than_one_launch(fh):
    # 33,000 queries: two launches of at most 32,768 query rows each; every output.
    oracle.set_threads(oracle_threads())
    L = 33000
    q = gen.normal(L * 16 * 64, 1.0, 50)
    k = gen.normal(L * 16 * 64, 1.0, 51)
    v = gen.normal(L * 8 * 64, 1.0, 52)
    sinks = gen.uniform(16, -2.0, 2.0, 53)
    got = run(fh, q, k, v, sinks, L, (0, 0, 2048), fh.PrefillOptions())
    assert np.all(np.isfinite(got))
    close(got, oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, 0, 2048, sinks))


def attention_f64(q, k, v, L, n_heads, n_kv, image, sinks):
    """The exact attention of a pure prefill in float64: scores q.k / 8 over
    the keys a query sees (causal, plus the whole image for image queries),
    softmax, times V, scaled by 1 / (1 + exp(sink - logsumexp))."""
    q = q.reshape(L, n_heads, 64).astype(np.float64)
    k = k.reshape(L, n_heads, 64).astype(np.float64)
    v = v.reshape(L, n_kv, 64).astype(np.float64)
    i, j = np.arange(L)[:, None], np.arange(L)[None, :]
    in_image = lambda x: (x >= image[0]) & (x < image[1])
    visible = (j <= i) | (in_image(i) & in_image(j))
    out = np.empty((L, n_heads, 64))
    for h in range(n_heads):
        s = np.where(visible, q[:, h] @ k[:, h].T / 8.0, -np.inf)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        den = p.sum(axis=1, keepdims=True)
        lse = m + np.log(den)
        out[:, h] = (p @ v[:, h // (n_heads // n_kv)]) / den / (1.0 + np.exp(sinks[h] - lse))
    return out


def test_split_products_error_is_fp32_level(fh):
    # Against the exact attention (float64, exact exp): the split products'
    # error is of the order of the FP32 matrix-core products' (both within the
    # FP32 bound above), max and mean.
    L, image = 1000, (0, 300)
    q = gen.normal(L * 16 * 64, 1.0, 60)
    k = gen.normal(L * 16 * 64, 1.0, 61)
    v = gen.normal(L * 8 * 64, 1.0, 62)
    sinks = gen.uniform(16, -2.0, 2.0, 63)
    exact = attention_f64(q, k, v, L, 16, 8, image, sinks.astype(np.float64))
    err = {}
    for products in ("split", "fp32"):
        opts = fh.PrefillOptions(exp=fh.ExpMode.EXACT, split_products=products == "split")
        d = np.abs(run(fh, q, k, v, sinks, L, (0, *image), opts).astype(np.float64) - exact)
        err[products] = (float(d.max()), float(d.mean()))
    assert err["split"][0] <= 2 * err["fp32"][0] and err["split"][1] <= 2 * err["fp32"][1], err


def test_split_products_take_pure_prefills_only(fh):
    # A prefill over generated keys, or one that starts past key 0, is refused
    # by the split entry point (nothing written) and taken by the FP32 one.
    import torch

    L, prefix, total = 40, 40, 48
    q = to_dev(gen.att_values(L * 16 * 64, 71, 3.0))
    pk = to_dev(gen.att_values(prefix * 16 * 64, 83, 3.0))
    gk = to_dev(gen.att_values((total - prefix) * 8 * 64, 37, 3.0))
    v = to_dev(gen.att_values(total * 8 * 64, 117, 3.0))
    sinks = to_dev(gen.att_values(16, 29, 2.0))
    out = torch.full((L * 16 * 64,), 7.0, device=q.device)
    ctx = fh.default_context()
    for qlen, prefix_len, total_len, offset in ((L, prefix, total, 8), (L - 8, prefix, prefix, 8)):
        rc = fh.lib().focr_attention_prefill_split(ctx.handle, q.data_ptr(), pk.data_ptr(), gk.data_ptr(),
                                                   v.data_ptr(), qlen, prefix_len, total_len, 16, 8, 64, offset, 1,
                                                   20, sinks.data_ptr(), 0, 0, out.data_ptr())
        assert rc == fh.FOCR_E_UNSUPPORTED
    torch.cuda.synchronize()
    assert bool(torch.all(out == 7.0))


def test_split_products_power_of_two_scaling_is_exact(fh):
    # The FP16 pairs scale every block by a power of two: Q x 2^-40 with
    # K x 2^40 leaves every score exact, V x 2^-60 scales every output by
    # exactly 2^-60, so the outputs are bitwise 2^-60 times the unscaled ones
    # (online and static, one work item and split key ranges).
    L, image = 1400, (0, 300)
    q = gen.normal(L * 16 * 64, 1.0, 70)
    k = gen.normal(L * 16 * 64, 1.0, 71)
    v = gen.normal(L * 8 * 64, 1.0, 72)
    sinks = gen.uniform(16, -2.0, 2.0, 73)
    for static in (False, True):
        if static:
            q, k = gen.normalized(L * 16 * 64, 74), gen.normalized(L * 16 * 64, 75)
        opts = fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE)
        base = run(fh, q, k, v, sinks, L, (0, *image), opts)
        scaled = run(fh, np.ldexp(q, -40), np.ldexp(k, 40), np.ldexp(v, -60), sinks, L, (0, *image), opts)
        assert np.all(np.isfinite(base))
        assert np.array_equal(np.ldexp(scaled, 60).view(np.uint32), base.view(np.uint32)), static


def test_split_products_wide_magnitudes(fh):
    # Rows of Q and K scaled by 2^u, u uniform in [-30, 0], and value dims by
    # 2^w, w uniform in [-30, 30]: every output dim within 1e-5 of the
    # oracle relative to that dim's largest output.
    L, image = 600, (0, 128)
    rng = np.random.default_rng(76)
    q = (gen.normal((L, 16, 64), 1.0, 77) * np.ldexp(1.0, rng.integers(-30, 1, (L, 16, 1)))).astype(np.float32)
    k = (gen.normal((L, 16, 64), 1.0, 78) * np.ldexp(1.0, rng.integers(-30, 1, (L, 16, 1)))).astype(np.float32)
    v = (gen.normal((L, 8, 64), 1.0, 79) * np.ldexp(1.0, rng.integers(-30, 31, (1, 8, 64)))).astype(np.float32)
    sinks = gen.uniform(16, -2.0, 2.0, 80)
    q, k, v = q.ravel(), k.ravel(), v.ravel()
    got = run(fh, q, k, v, sinks, L, (0, *image), fh.PrefillOptions())
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, *image, sinks, exp_fast=True).reshape(L, 16, 64)
    scale = np.max(np.abs(want), axis=0, keepdims=True)
    assert np.all(np.abs(got - want) <= 1e-5 * scale), float(np.max(np.abs(got - want) / scale))


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_tiny_and_subnormal_magnitudes(fh, static, products):
    # Q times 2^124 against K times 2^-124 (scores of order one from keys
    # that are tiny normals and, one in five or so, subnormals), and value
    # dims from 2^-145 to 2^20. Against the exact attention of these inputs
    # (float64): every output within 1e-5 of its dim's largest output, plus,
    # in the subnormal range, a few steps of 2^-149 for the FP16-pair products
    # (the output's last roundings) and one step per key for the FP32 ones
    # (their P V products round there one by one, as the reference's do).
    L, image = 700, (0, 128)
    if static:
        q, k = gen.normalized(L * 16 * 64, 84), gen.normalized(L * 16 * 64, 85)
    else:
        q, k = gen.normal(L * 16 * 64, 1.0, 84), gen.normal(L * 16 * 64, 1.0, 85)
    q = (q * np.float32(2.0 ** 124)).astype(np.float32)
    k = (k * np.float32(2.0 ** -124)).astype(np.float32)
    dims = np.ldexp(1.0, np.tile([0, -110, -120, -126, -130, -140, -145, 20], 8))
    v = (gen.normal((L, 8, 64), 1.0, 86) * dims).astype(np.float32).ravel()
    sinks = gen.uniform(16, -2.0, 2.0, 87)
    assert np.all(np.isfinite(q)) and np.any((k != 0) & (np.abs(k) < 2.0 ** -126))
    opts = fh.PrefillOptions(exp=fh.ExpMode.FAST if static else fh.ExpMode.EXACT,
                             fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE,
                             split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, *image), opts).astype(np.float64)
    exact = attention_f64(q, k, v, L, 16, 8, image, sinks.astype(np.float64))
    scale = np.max(np.abs(exact), axis=0, keepdims=True)
    steps = 8 if products == "split" else L + 8
    bound = 1e-5 * scale + steps * 2.0 ** -149
    assert np.all(np.abs(got - exact) <= bound), float(np.max((np.abs(got - exact) - bound) / scale))


@pytest.mark.parametrize("static", [False, True])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_nan_key_propagates_as_the_reference(fh, static, products):
    # static_shift/tests.rs:311-367 (nan_keys_propagate_in_masked_tiles): a
    # NaN in head 0 of key 66, text after the image [3, 65): rows 66 to 69
    # see it and are NaN in head 0; rows 64 and 65 mask it and stay finite,
    # as does every other head.
    L, image = 70, (3, 65)
    q = gen.normalized(L * 16 * 64, 91)
    k = gen.normalized(L * 16 * 64, 92)
    v = gen.values(L * 8 * 64, 93, 3.0)
    sinks = gen.values(16, 94, 2.0)
    k[66 * 16 * 64] = np.nan
    opts = fh.PrefillOptions(fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE,
                             split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, *image), opts)
    poisoned = np.zeros((L, 16), bool)
    poisoned[66:, 0] = True
    assert np.array_equal(np.isnan(got).all(axis=2), poisoned)
    assert np.array_equal(np.isnan(got).any(axis=2), poisoned)
    want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, *image, sinks, static=static).reshape(L, 16, 64)
    close(got[~poisoned], want[~poisoned])


@pytest.mark.parametrize("static,exp", [(False, "fast"), (False, "exact"), (True, "fast")])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_nonfinite_query_poisons_its_row_and_head_only(fh, static, exp, products):
    # An infinity or NaN in one query value makes that query's scores in its
    # head infinite or NaN; the reference's output for that (row, head) is
    # all NaN (exp(inf - inf), or 0 / 0 when every score is -inf), and no
    # other output changes. Rows in and past the image, tiles split into
    # several key ranges.
    L, image = 2100, (0, 700)
    q = gen.normalized(L * 16 * 64, 121) if static else gen.normal(L * 16 * 64, 1.0, 121)
    k = gen.normalized(L * 16 * 64, 122) if static else gen.normal(L * 16 * 64, 1.0, 122)
    v = gen.normal(L * 8 * 64, 1.0, 123)
    sinks = gen.uniform(16, -2.0, 2.0, 124)
    poisoned = np.zeros((L, 16), bool)
    for r, h, d, val in ((40, 3, 5, np.inf), (600, 2, 63, -np.inf), (1800, 7, 0, np.nan), (2000, 11, 9, np.inf)):
        q[(r * 16 + h) * 64 + d] = val
        poisoned[r, h] = True
    opts = fh.PrefillOptions(exp=fh.ExpMode.FAST if exp == "fast" else fh.ExpMode.EXACT,
                             fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE,
                             split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, *image), opts)
    oracle.set_threads(oracle_threads())
    if exp == "fast":
        want = oracle.attention_prefill_fast(q, k, v, L, L, L, 16, 8, 0, *image, sinks, static=static)
    else:
        want = oracle.attention_prefill(q, k, v, L, L, L, 16, 8, 0, *image, sinks, exp_fast=False)
    want = want.reshape(L, 16, 64)
    assert np.array_equal(np.isnan(want).all(axis=2), poisoned) and np.all(np.isfinite(want[~poisoned]))
    assert np.array_equal(np.isnan(got).all(axis=2), poisoned)
    assert np.all(np.isfinite(got[~poisoned]))
    close(got[~poisoned], want[~poisoned])


@pytest.mark.parametrize("case", ["k_neg_inf", "k_pos_inf", "v_inf"])
def test_split_products_nonfinite_kv_take_the_fp32_products(fh, case):
    # An infinity in an FP16 pair meets zero halves (0 * inf = NaN) where the
    # FP32 products give +-inf, so a call whose K or V holds a non-finite
    # value runs the FP32 products on the device: the outputs are bitwise the
    # FP32 entry point's (the same plan), and for V, and for K under the
    # online softmax, the NaN and infinity patterns and the finite values are
    # the oracle's (a -inf score is a zero probability; an infinite value
    # reaches the rows that see its key as an infinity, and as a NaN, 0 * inf,
    # the earlier rows of the 32-row group that multiply the key's masked zero
    # probability; the static softmax's exp takes finite scores only,
    # exp_lanes in static_shift.rs). The next finite call takes the pairs
    # again.
    L, image = 300, (0, 100)
    q = gen.normalized(L * 16 * 64, 95)
    k = gen.normalized(L * 16 * 64, 96)
    v = gen.values(L * 8 * 64, 97, 3.0)
    sinks = gen.values(16, 98, 2.0)
    clean = run(fh, q, k, v, sinks, L, (0, *image), fh.PrefillOptions())
    bad_k, bad_v = k.copy(), v.copy()
    if case == "v_inf":
        bad_v[(150 * 8 + 3) * 64 + 7] = np.inf
    else:
        bad_k[(150 * 16 + 6) * 64] = -np.inf if case == "k_neg_inf" else np.inf
    for static in (False, True):
        opts = dict(fp32_softmax=fh.Softmax.STATIC if static else fh.Softmax.ONLINE)
        split = run(fh, q, bad_k, bad_v, sinks, L, (0, *image), fh.PrefillOptions(**opts))
        fp32 = run(fh, q, bad_k, bad_v, sinks, L, (0, *image), fh.PrefillOptions(split_products=False, **opts))
        assert not np.all(np.isfinite(split))
        assert np.array_equal(split, fp32, equal_nan=True), static
        if case == "v_inf" or not static:
            want = oracle.attention_prefill(q, bad_k, bad_v, L, L, L, 16, 8, 0, *image, sinks,
                                            static=static).reshape(L, 16, 64)
            assert np.array_equal(np.isnan(split), np.isnan(want)) and np.array_equal(np.isinf(split), np.isinf(want))
            fin = np.isfinite(want)
            if case != "v_inf":
                assert np.any(fin[150:, 6]) and not np.all(fin[150:, 6])
            close(split[fin], want[fin])
    again = run(fh, q, k, v, sinks, L, (0, *image), fh.PrefillOptions())
    assert np.array_equal(again.view(np.uint32), clean.view(np.uint32))


@pytest.mark.parametrize("n_heads,n_kv", [(16, 16), (16, 4), (4, 1)])
@pytest.mark.parametrize("L,image", [(4, (0, 4)), (33, (1, 20)), (700, (0, 300))])
@pytest.mark.parametrize("products", ["split", "fp32"])
def test_gqa_groupings(fh, n_heads, n_kv, L, image, products):
    # Head groupings other than the checkpoint's 16 / 8 (prefill64 takes any
    # n_heads divisible by n_kv_heads), the smallest prefill the tiles take
    # (4 rows) and a split plan; online, Fast exp.
    q = gen.att_values(L * n_heads * 64, 111 + L, 3.0)
    k = gen.att_values(L * n_heads * 64, 113 + L, 3.0)
    v = gen.att_values(L * n_kv * 64, 117 + L, 3.0)
    sinks = gen.att_values(n_heads, 119, 2.0)
    opts = fh.PrefillOptions(split_products=products == "split")
    got = run(fh, q, k, v, sinks, L, (0, *image), opts, n_heads=n_heads, n_kv=n_kv)
    want = oracle.attention_prefill(q, k, v, L, L, L, n_heads, n_kv, 0, *image, sinks, exp_fast=True)
    close(got, want.reshape(L, n_heads, 64))
