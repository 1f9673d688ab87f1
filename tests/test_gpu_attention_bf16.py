"""BF16 prefill attention (A8) on the GPU against the oracle, within the BF16
tolerance: max|d| / max|ref| <= 2e-3, and within the reference's own f64
bound on BF16-rounded operands (prefill64/bf16.rs matches_bf16_operand_reference,
bf16/static_shift/tests.rs)."""
import numpy as np
import pytest

import gen
import oracle
from gpu_util import host, max_rel, to_dev
from test_oracle_bf16 import CASES, f64_attention

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fh():
    import focr_hip

    return focr_hip


def run(fh, q, k, v, sinks, L, image, softmax, heads=16, kv_heads=8):
    import torch

    out = torch.full((L * heads * 64,), float("nan"), device="cuda")
    kv = fh.CompactKv.prefill(to_dev(k), to_dev(v), L, heads, kv_heads)
    ran = fh.attention_prefill_bf16(to_dev(q), kv, L, fh.Geometry(0, *image), to_dev(sinks), out,
                                    fh.PrefillOptions(softmax=softmax))
    assert ran
    return host(out).reshape(L, heads, 64)


@pytest.mark.parametrize("L,image_start,image_end", CASES + [(600, 0, 0), (33, 0, 33)])
def test_online_bf16(fh, L, image_start, image_end):
    r = oracle.bf16_round
    q = r(gen.values(L * 16 * 64, 17 + L, 3.0))
    k = r(gen.values(L * 16 * 64, 19 + L, 3.0))
    v = r(gen.values(L * 8 * 64, 23 + L, 3.0))
    sinks = gen.values(16, 29, 2.0)
    got = run(fh, q, k, v, sinks, L, (image_start, image_end), fh.Softmax.ONLINE)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, image_start, image_end, sinks, static=False)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 2e-3
    exact = f64_attention(q, k, v, L, 16, 8, image_start, image_end, sinks)
    assert np.abs(got - exact).max() <= 3.0 * 2.0 ** -9 + 2e-3


@pytest.mark.parametrize("L,image_start,image_end", CASES + [(600, 0, 0)])
def test_static_bf16(fh, L, image_start, image_end):
    r = oracle.bf16_round
    q = r(gen.normalized(L * 16 * 64, 17 + L))
    k = r(gen.normalized(L * 16 * 64, 19 + L))
    v = r(gen.values(L * 8 * 64, 23 + L, 3.0))
    sinks = gen.values(16, 29, 2.0)
    got = run(fh, q, k, v, sinks, L, (image_start, image_end), fh.Softmax.STATIC)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, image_start, image_end, sinks, static=True)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 2e-3
    exact = f64_attention(q, k, v, L, 16, 8, image_start, image_end, sinks, shift=False)
    assert np.abs(got - exact).max() <= 3.0 * 2.0 * (2.0 ** -8 + 7.5e-5) + 1e-4


@pytest.mark.parametrize("L,image", [(130, (2, 100)), (97, (0, 40)), (66, (3, 65)), (33, (0, 0)), (300, (5, 262)),
                                     (259, (0, 257)), (6, (0, 3))])
def test_unrounded_operands_online(fh, L, image):
    # FP32 operands: the kernel rounds Q, K, V itself, like the reference, and
    # the reference's short key tiles (and rows of a last one- or two-query
    # tile) take the FP32 path on the unrounded values.
    q = gen.values(L * 16 * 64, 3 + L, 3.0)
    k = gen.values(L * 16 * 64, 4 + L, 3.0)
    v = gen.values(L * 8 * 64, 5 + L, 3.0)
    sinks = gen.values(16, 29, 2.0)
    got = run(fh, q, k, v, sinks, L, image, fh.Softmax.ONLINE)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, image[0], image[1], sinks, static=False)
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 2e-3


@pytest.mark.parametrize("L,image", [(130, (2, 100)), (66, (3, 65))])
def test_unrounded_operands_static(fh, L, image):
    q = gen.normalized(L * 16 * 64, 3 + L)
    k = gen.normalized(L * 16 * 64, 4 + L)
    v = gen.values(L * 8 * 64, 5 + L, 3.0)
    sinks = gen.values(16, 29, 2.0)
    got = run(fh, q, k, v, sinks, L, image, fh.Softmax.STATIC)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, image[0], image[1], sinks, static=True)
    assert max_rel(got, want) <= 2e-3


def test_unsupported_shapes_write_nothing(fh):
    import torch

    L = 3
    q = to_dev(gen.values(L * 16 * 64, 1))
    v = to_dev(gen.values(L * 8 * 64, 2))
    out = torch.full((L * 16 * 64,), 7.0, device="cuda")
    kv = fh.CompactKv.prefill(q, v, L, 16, 8)
    assert not fh.attention_prefill_bf16(q, kv, L, fh.Geometry(0, 0, 0), to_dev(gen.values(16, 3)), out)
    mixed = fh.CompactKv(q, q, v, 2, 3, 16, 8, 64)
    assert not fh.attention_prefill_bf16(q, mixed, L, fh.Geometry(0, 0, 0), to_dev(gen.values(16, 3)), out)
    assert bool(torch.all(out == 7.0))


@pytest.mark.parametrize("softmax", ["online", "static"])
def test_config4_full_page_bf16(fh, softmax):
    # BASELINE config 4 shape (6,544 tokens, image prefix 4,096), Q/K/V ~ N(0,1),
    # checked against the oracle on query tiles that span the image end.
    L, image_end = 6544, 4096
    q = gen.normal(L * 16 * 64, 1.0, 20)
    k = gen.normal(L * 16 * 64, 1.0, 21)
    v = gen.normal(L * 8 * 64, 1.0, 22)
    sinks = gen.uniform(16, -2.0, 2.0, 23)
    sm = fh.Softmax.ONLINE if softmax == "online" else fh.Softmax.STATIC
    got = run(fh, q, k, v, sinks, L, (0, image_end), sm)
    assert np.all(np.isfinite(got))
    for lo, hi in ((0, 2), (127, 129), (203, 205)):
        want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, 0, image_end, sinks, static=softmax == "static",
                                             tiles=(lo, hi))
        rows = slice(32 * lo, 32 * hi)
        assert max_rel(got[rows], want[rows]) <= 2e-3


@pytest.mark.parametrize("softmax", ["online", "static"])
@pytest.mark.parametrize("L,image", [(3001, (0, 1500)), (2562, (0, 0))])
def test_split_key_ranges_bf16(fh, softmax, L, image):
    # Query tiles with more than 1,024 visible keys run as several work items
    # (whole 128-key tiles) merged afterwards; L % 32 = 1 or 2 keeps the
    # short-rows kernel's rows out of the merge.
    oracle.set_threads(8)
    r = oracle.bf16_round
    q = r(gen.normalized(L * 16 * 64, 401))
    k = r(gen.normalized(L * 16 * 64, 402))
    v = r(gen.values(L * 8 * 64, 403, 3.0))
    sinks = gen.values(16, 29, 2.0)
    sm = fh.Softmax.STATIC if softmax == "static" else fh.Softmax.ONLINE
    got = run(fh, q, k, v, sinks, L, image, sm)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, *image, sinks, static=softmax == "static")
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) <= 2e-3


@pytest.mark.parametrize("softmax", ["online", "static"])
def test_nonfinite_inputs_poison_what_the_reference_poisons(fh, softmax):
    # An infinity or NaN in one query value poisons that (row, head); a NaN
    # key value poisons its head's rows that see the key (causal after it,
    # and every image row for an image key); all of them all NaN, as the
    # reference's BF16 tiles give, and every other output unchanged. Tiles
    # split into several key ranges.
    oracle.set_threads(8)
    r = oracle.bf16_round
    L, image = 2100, (0, 700)
    q = r(gen.normalized(L * 16 * 64, 131))
    k = r(gen.normalized(L * 16 * 64, 132))
    v = r(gen.values(L * 8 * 64, 133, 3.0))
    sinks = gen.values(16, 29, 2.0)
    for row, h, d, val in ((40, 3, 5, np.inf), (1800, 7, 0, np.nan), (600, 2, 63, -np.inf)):
        q[(row * 16 + h) * 64 + d] = val
    k[(1500 * 16 + 9) * 64 + 4] = np.nan  # text key 1500, head 9
    k[(650 * 16 + 12) * 64 + 1] = np.nan  # image key 650, head 12
    poisoned = np.zeros((L, 16), bool)
    poisoned[40, 3] = poisoned[1800, 7] = poisoned[600, 2] = True
    poisoned[1500:, 9] = True
    poisoned[:, 12] = True
    static = softmax == "static"
    got = run(fh, q, k, v, sinks, L, image, fh.Softmax.STATIC if static else fh.Softmax.ONLINE)
    want = oracle.attention_prefill_bf16(q, k, v, L, 16, 8, *image, sinks, static=static).reshape(L, 16, 64)
    assert np.array_equal(np.isnan(want).all(axis=2), poisoned) and np.all(np.isfinite(want[~poisoned]))
    assert np.array_equal(np.isnan(got).all(axis=2), poisoned)
    assert np.all(np.isfinite(got[~poisoned]))
    assert max_rel(got[~poisoned], want[~poisoned]) <= 2e-3
