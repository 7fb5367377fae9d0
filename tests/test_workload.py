"""CPU tests of the prefill benchmark's routing workload (512 tokens, expert popularity
Zipf(1.2) over 512 experts, hot experts with more than 100 tokens and many with none).  The fitted router bias is
run through the test oracle's own router (device-order bf16 products, top-10 routing) on a synthetic layer's
router weights and N(0, 1) tokens, as the benchmark and the parity test run it."""
import numpy as np

import oracle as O
import stratametal_amd as S


def test_zipf_targets_closed_form():
    c = S.zipf_targets(512, 1.2, 512, 10)
    assert abs(c.sum() - 5120) < 1e-6
    assert c.max() == 512 and (c <= 512).all()
    free = np.nonzero(c < 512)[0]
    r = free + 1.0
    # uncapped ranks follow C * r^-1.2 exactly: consecutive ratios are ((r + 1) / r)^1.2
    np.testing.assert_allclose(c[free[:-1]] / c[free[1:]], ((r[1:]) / r[:-1]) ** 1.2, rtol=1e-12)


def test_zipf_routing_follows_zipf_1_2():
    g = O.Geom()
    H, E, T, K = g.n_embd, g.n_expert, 512, g.top_k
    bias = S.zipf_bias(E, 1.2, seed=1001, n_tokens=T, top_k=K, n_embd=H)
    W = O.gen_bf16(4242, 4, E * H, 0.02)  # a synthetic layer's router (stream 4), as the device generates it
    x = O.gen_normal(17, 100, T * H).reshape(T, H)
    xb = O.bf16_from_f32(x)
    logits = np.stack([O.bf16_gemv_dev(xb[t], W, H, E) for t in range(T)]) + bias[None, :]
    ids, _ = O.route_dev(logits.astype(np.float32), K)
    counts = np.bincount(ids.ravel(), minlength=E)
    D = int((counts > 0).sum())
    assert 300 <= D <= 450, D
    assert counts.max() > 100 and (counts == 0).sum() >= 30
    srt = np.sort(counts)[::-1]
    rank = np.arange(1, E + 1)
    m = (srt > 0) & (srt < T)
    slope = np.polyfit(np.log(rank[m]), np.log(srt[m]), 1)[0]
    assert abs(slope + 1.2) <= 0.1, slope
    # the popularity order is the seeded permutation's: the bias orders the experts' mean counts
    hot = np.argsort(-bias)[:20]
    assert counts[hot].mean() > 10 * counts.mean()


def test_zipf_bias_is_deterministic_and_seeded():
    a = S.zipf_bias(512, 1.2, 5)
    assert np.array_equal(a, S.zipf_bias(512, 1.2, 5))
    assert not np.array_equal(a, S.zipf_bias(512, 1.2, 6))
    # another seed permutes the ranks: the hottest experts differ
    assert set(np.argsort(-a)[:5]) != set(np.argsort(-S.zipf_bias(512, 1.2, 6))[:5])
