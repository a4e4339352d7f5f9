"""The oracle's lambdarank restatement (objective/lambdarank.rs) against the reference's own tests of it
(lambdarank.rs:420-783): an independent transcription of LightGBM 3.3.5 `GetGradientsForOneQuery` (pair loop order,
sigmoid table and discounts written out here from LightGBM's definitions) over the reference's 400 xorshift cases
and its 120k-row query, to the reference's tolerance; the sigmoid table and max DCG at known values; -inf scores."""

import math

import numpy as np

import oracle

M64 = (1 << 64) - 1
LABEL_GAIN = [float((1 << i) - 1) for i in range(31)]  # config.rs:118-121


class Xorshift:
    """xorshift64* of lambdarank.rs:424-442."""

    def __init__(self, seed):
        self.s = seed

    def next(self):
        s = self.s
        s ^= s >> 12
        s ^= (s << 25) & M64
        s ^= s >> 27
        self.s = s
        return (s * 0x2545F4914F6CDD1D) & M64

    def below(self, n):
        return self.next() % n

    def unit(self):
        return np.float32(self.next() >> 40) / np.float32(1 << 24)


def random_case(rng, index):
    """lambdarank.rs:531-555."""
    cnt = 1 + rng.below(60)
    label = np.array([rng.below(5) for _ in range(cnt)], np.float32)
    if index % 4 == 0:
        score = np.zeros(cnt, np.float32)
    elif index % 4 == 1:
        score = np.array([np.float32(rng.below(4)) * np.float32(0.5) for _ in range(cnt)], np.float32)
    else:
        score = np.array([(rng.unit() - np.float32(0.5)) * np.float32(8.0) for _ in range(cnt)], np.float32)
    weight = None
    if index % 3 == 0:
        weight = np.array([np.float32(0.5) + rng.unit() for _ in range(cnt)], np.float32)
    return label, score, weight, [1, 3, 10, 30, 1000][index % 5], index % 7 != 6


def discount(rank):
    return 1.0 / math.log2(2.0 + rank)  # DCGCalculator::GetDiscount


def lightgbm_sigmoid(sigmoid):
    """ConstructSigmoidTable / GetSigmoid, entries computed where they are read."""
    lo, hi = -50.0 / sigmoid / 2.0, 50.0 / sigmoid / 2.0
    factor = (1024.0 * 1024.0) / (hi - lo)

    def entry(i):
        return 1.0 / (1.0 + math.exp((i / factor + lo) * sigmoid))

    def get(x):
        if x <= lo:
            return entry(0)
        if x >= hi:
            return entry(1024 * 1024 - 1)
        return entry(int((x - lo) * factor))

    return get


def max_dcg(k, labels):
    """DCGCalculator::CalMaxDCGAtK."""
    count = [0] * len(LABEL_GAIN)
    for l in labels:
        count[int(l)] += 1
    top, dcg = len(LABEL_GAIN) - 1, 0.0
    for j in range(min(k, len(labels))):
        while top > 0 and count[top] == 0:
            top -= 1
        dcg += discount(j) * LABEL_GAIN[top]
        count[top] -= 1
    return dcg


def lightgbm_query(label, score, weight, inverse_max_dcg, sigmoid, norm, truncation):
    """GetGradientsForOneQuery and RankingObjective's weight loop (lambdarank.rs:444-528), f64 sums."""
    cnt = len(label)
    get = lightgbm_sigmoid(sigmoid)
    s = [float(v) for v in score]
    lam, hes = [0.0] * cnt, [0.0] * cnt
    idx = sorted(range(cnt), key=lambda a: -s[a])
    best = s[idx[0]]
    w = cnt - 1
    if w > 0 and s[idx[w]] == -math.inf:
        w -= 1
    worst = s[idx[w]]
    total, i = 0.0, 0
    while i + 1 < cnt and i < truncation:
        if s[idx[i]] == -math.inf:
            i += 1
            continue
        for j in range(i + 1, cnt):
            if s[idx[j]] == -math.inf or label[idx[i]] == label[idx[j]]:
                continue
            hr, lr = (i, j) if label[idx[i]] > label[idx[j]] else (j, i)
            high, low = idx[hr], idx[lr]
            delta = s[high] - s[low]
            gap = LABEL_GAIN[int(label[high])] - LABEL_GAIN[int(label[low])]
            pd = abs(discount(hr) - discount(lr))
            dn = gap * pd * inverse_max_dcg
            if norm and best != worst:
                dn /= float(np.float32(0.01)) + abs(delta)
            pl = get(delta)
            ph = pl * (1.0 - pl)
            pl *= -sigmoid * dn
            ph *= sigmoid * sigmoid * dn
            lam[low] -= pl
            hes[low] += ph
            lam[high] += pl
            hes[high] += ph
            total -= 2.0 * pl
        i += 1
    if norm and total > 0.0:
        f = math.log2(1.0 + total) / total
        lam = [v * f for v in lam]
        hes = [v * f for v in hes]
    if weight is not None:
        lam = [v * float(weight[j]) for j, v in enumerate(lam)]
        hes = [v * float(weight[j]) for j, v in enumerate(hes)]
    return np.array(lam), np.array(hes)


def assert_close(got, want, what):
    # lambdarank.rs:565-575
    scale = np.abs(want).max() if len(want) else 0.0
    tol = 1e-6 * np.maximum(np.abs(want), scale * 1e-3) + 1e-30
    bad = np.abs(got.astype(np.float64) - want) > tol
    assert not bad.any(), (what, np.flatnonzero(bad)[:5], got[bad][:5], want[bad][:5])


def test_gradients_match_the_lightgbm_pair_loop():
    # lambdarank.rs:577-611
    rng = Xorshift(0x9E3779B97F4A7C15)
    for index in range(400):
        label, score, weight, trunc, norm = random_case(rng, index)
        md = max_dcg(trunc, label)
        inv = 1.0 / md if md > 0.0 else 0.0
        assert oracle.max_dcg_at_k(trunc, label, LABEL_GAIN) == md
        want_g, want_h = lightgbm_query(label, score, weight, inv, 1.3, norm, trunc)
        g, h = oracle.lambdarank_query(score, label, LABEL_GAIN, inv, 1.3, norm, trunc, weight)
        assert_close(g, want_g, f"case {index} gradient")
        assert_close(h, want_h, f"case {index} hessian")


def test_huge_query_matches_the_pair_loop():
    # lambdarank.rs:613-660: 120k rows, truncation 30; rows ranked below 100 or at multiples of 997 compared. The
    # pair loop is vectorized over j here (the tolerance does not depend on the order of the adds)
    rng = Xorshift(0x5EED)
    cnt = 120_000
    label = np.array([rng.below(5) for _ in range(cnt)], np.float32)
    score = np.array([(rng.unit() - np.float32(0.5)) * np.float32(8.0) for _ in range(cnt)], np.float32)
    inv = 1.0 / max_dcg(30, label)
    g, h = oracle.lambdarank_query(score, label, LABEL_GAIN, inv, 1.3, True, 30)
    s = score.astype(np.float64)
    idx = np.argsort(-s, kind="stable")
    ranked_s, ranked_l = s[idx], label[idx]
    gain = np.array(LABEL_GAIN)[ranked_l.astype(int)]
    disc = 1.0 / np.log2(2.0 + np.arange(cnt))
    lo, hi = -50.0 / 1.3 / 2.0, 50.0 / 1.3 / 2.0
    factor = (1024.0 * 1024.0) / (hi - lo)
    entry = lambda i: 1.0 / (1.0 + np.exp((i / factor + lo) * 1.3))  # noqa: E731
    lam, hes = np.zeros(cnt), np.zeros(cnt)
    total = 0.0
    by_distance = ranked_s[0] != ranked_s[-1]
    for i in range(30):
        j = np.arange(i + 1, cnt)
        j = j[ranked_l[j] != ranked_l[i]]
        sign = np.where(ranked_l[i] > ranked_l[j], 1.0, -1.0)
        delta = sign * (ranked_s[i] - ranked_s[j])
        dn = sign * (gain[i] - gain[j]) * np.abs(disc[i] - disc[j]) * inv
        if by_distance:
            dn = dn / (float(np.float32(0.01)) + np.abs(delta))
        k = np.clip(((delta - lo) * factor).astype(np.int64), 0, 1024 * 1024 - 1)
        p = np.where(delta <= lo, entry(0), np.where(delta >= hi, entry(1024 * 1024 - 1), entry(k)))
        pl = p * (-1.3 * dn)
        ph = p * (1.0 - p) * (1.3 * 1.3 * dn)
        lam[i] += (sign * pl).sum()
        np.subtract.at(lam, j, sign * pl)
        hes[i] += ph.sum()
        np.add.at(hes, j, ph)
        total -= 2.0 * pl.sum()
    f = math.log2(1.0 + total) / total
    rank = np.arange(cnt)
    pick = (rank < 100) | (rank % 997 == 0)
    assert_close(g[idx][pick], lam[pick] * f, "gradient")
    assert_close(h[idx][pick], hes[pick] * f, "hessian")


def test_min_score_items_get_no_pairs():
    # lambdarank.rs:662-700
    label = np.array([2.0, 0.0, 1.0, 0.0], np.float32)
    score = np.array([0.5, -np.inf, -0.2, 0.1], np.float32)
    md = max_dcg(30, label)
    g, h = oracle.lambdarank_query(score, label, LABEL_GAIN, 1.0 / md, 1.3, True, 30)
    assert (g[1], h[1]) == (0.0, 0.0)
    want_g, want_h = lightgbm_query(label, score, None, 1.0 / md, 1.3, True, 30)
    assert_close(g, want_g, "gradient")
    assert_close(h, want_h, "hessian")


def test_sigmoid_table_follows_lightgbm():
    # lambdarank.rs:702-725
    sig = 2.0
    lo, hi = -50.0 / sig / 2.0, 50.0 / sig / 2.0
    want = lightgbm_sigmoid(sig)
    for x in [-100.0, lo, -3.7, -1e-9, 0.0, 1e-9, 0.25, 4.0, hi - 1e-12, hi, 30.0]:
        assert oracle.lib().oracle_sigmoid_table_get(sig, x) == want(x), x
    assert abs(oracle.lib().oracle_sigmoid_table_get(sig, 0.0) - 0.5) < 1e-4


def test_max_dcg_follows_lightgbm():
    # lambdarank.rs:727-735
    gain = [0.0, 1.0, 3.0, 7.0]
    assert oracle.max_dcg_at_k(3, [1.0, 3.0, 0.0, 2.0, 3.0], gain) == 7.0 * discount(0) + 7.0 * discount(1) + \
        3.0 * discount(2)
    assert oracle.max_dcg_at_k(3, [0.0, 0.0], gain) == 0.0
    assert oracle.max_dcg_at_k(10, [1.0], gain) == 1.0


def test_label_checks_follow_rusts_saturating_casts():
    # check_labels (lambdarank.rs:172-188) converts with Rust's `as`: NaN -> 0 and out-of-range values saturate, so a
    # NaN label passes all three checks (and takes label 0's gain), 3e9 saturates to i32::MAX and fails the integer
    # check, and -inf and +inf fail it too
    nan = float("nan")
    assert oracle.check_labels([0, 1, 4, 2], 5) == 0
    assert oracle.check_labels([0, nan, 3], 5) == 0
    assert oracle.check_labels([3e9], 5) == 1
    assert oracle.check_labels([float("-inf")], 5) == 1
    assert oracle.check_labels([float("inf")], 5) == 1
    assert oracle.check_labels([1.5], 5) == 1
    assert oracle.check_labels([-2.0], 5) == 2
    assert oracle.check_labels([5.0], 5) == 3
    assert oracle.check_labels([2.0e9], 5) == 3  # an integer in i32 range, past the gains
    # a NaN label takes label 0's gain (lambdarank.rs:349) and its pairs compare as NaN (:391-396): finite gradients
    scores = np.array([0.5, -1.0, 2.0, 0.1], np.float32)
    gn, hn = oracle.lambdarank_query(scores, [nan, 2, 1, 3], [0.0, 1.0, 3.0, 7.0], 0.1)
    assert np.isfinite(gn).all() and np.isfinite(hn).all()
