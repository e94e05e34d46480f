"""Pins oracle/layer_oracle.cpu_step (the configuration-3 checker) on
reduced shapes against an independent construction: numpy F64 products of
the decoded matrices, the GQA broadcast as np.repeat of whole KV heads
(query head h reads KV head h // group, backends/metal/kernels/attention.metal:40),
and SiLU as g * expit(g) (scipy's logistic; the reference's silu is
f32(x * logistic(x)) in F64, backends/cpu/vector.zig:177-196). A wrong head
mapping, a missing residual or a swapped gate/up pair each moves the
logits far beyond the GPU layer test's 2e-3 normwise bound on these seeds,
which the last test checks, so a shared mistake in the oracle and the product cannot pass the GPU layer test."""
import numpy as np
import pytest
from scipy.special import expit

import nuclis_amd as nq
from nuclis_amd.synth import gaussian
from oracle import layer_oracle
from oracle import oracle as orc

HIDDEN, KV_HEADS, GROUP, FFN, VOCAB = 512, 2, 6, 1024, 2048
Q_ROWS, KV_ROWS = KV_HEADS * GROUP * 128, KV_HEADS * 128
SHAPES = {
    "q": (12, Q_ROWS, HIDDEN, 40),
    "k": (12, KV_ROWS, HIDDEN, 41),
    "v": (12, KV_ROWS, HIDDEN, 42),
    "o": (12, HIDDEN, Q_ROWS, 43),
    "gate": (12, FFN, HIDDEN, 44),
    "up": (12, FFN, HIDDEN, 45),
    "down": (12, HIDDEN, FFN, 46),
    "lm_head": (14, VOCAB, HIDDEN, 47),
}


@pytest.fixture(scope="module")
def weights():
    return {n: nq.quantize(e, gaussian(s, (r, c), 0.02)) for n, (e, r, c, s) in SHAPES.items()}


def independent_step(weights, x, *, head_map="repeat", residual=True, swap_pair=False):
    dec = {n: orc.decode_matrix(e, weights[n], r, c).astype(np.float64) for n, (e, r, c, _) in SHAPES.items()}

    def mv(n, v):
        return (dec[n] @ np.asarray(v, np.float64)).astype(np.float32)

    v = mv("v", x).reshape(KV_HEADS, 128)
    if head_map == "repeat":
        attn = np.repeat(v, GROUP, axis=0).ravel()
    else:  # interleaved: query head h reads KV head h % KV_HEADS
        attn = np.tile(v, (GROUP, 1)).ravel()
    o = mv("o", attn)
    h1 = (x.astype(np.float64) + o).astype(np.float32) if residual else o
    g, u = mv("gate", h1), mv("up", h1)
    if swap_pair:
        g, u = u, g
    g64 = g.astype(np.float64)
    act = ((g64 * expit(g64)).astype(np.float32) * u).astype(np.float32)
    h2 = (h1.astype(np.float64) + mv("down", act)).astype(np.float32)
    return mv("lm_head", h2)


@pytest.mark.parametrize("seed", [50, 51, 52])
def test_cpu_step_matches_independent_construction(weights, seed):
    x = gaussian(seed, HIDDEN)
    got = layer_oracle.cpu_step(SHAPES, weights, x)
    want = independent_step(weights, x)
    # both sum in F64 and round each matvec once; only the summation order differs
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()
    assert orc.argmax(got) == int(np.argmax(want))


def test_silu_matches_expit_and_special_values():
    g = np.concatenate([np.linspace(-60, 60, 2001), [0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 1e30, -1e30]])
    g = g.astype(np.float32)
    want = (g.astype(np.float64) * expit(g.astype(np.float64))).astype(np.float32)
    np.testing.assert_array_equal(layer_oracle.silu(g), want)
    s = layer_oracle.silu(np.array([np.inf, -np.inf, np.nan], np.float32))
    assert s[0] == np.inf and s[1] == 0 and np.signbit(s[1]) and np.isnan(s[2])


@pytest.mark.parametrize("mutation", [dict(head_map="interleave"), dict(residual=False), dict(swap_pair=True)])
def test_plausible_mistakes_change_the_greedy_token(weights, mutation):
    """The layer check is sensitive: the GPU layer test asks for the same
    greedy token and logits within 2e-3 normwise; each mistake breaks both
    on every seed used above."""
    for seed in (50, 51, 52):
        x = gaussian(seed, HIDDEN)
        ref = layer_oracle.cpu_step(SHAPES, weights, x)
        bad = independent_step(weights, x, **mutation)
        assert np.abs(bad - ref).max() / np.abs(ref).max() > 2e-2
