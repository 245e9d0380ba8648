"""The oracle's sampling chain (oracle/g4o_sampler.c) pinned against the
reference's own sampler.c built in place (oracle/_ref, same IEEE flags): the
drawn ids, the logits each call rewrites and the RNG words are compared bit for
bit over seeded runs.  Closed-form checks hold without that build: greedy is
the first argmax, top_k = 1 is the argmax whatever the RNG, the RNG's seeding
reproduces the published splitmix64 words, and draw frequencies follow the
softmax of two tokens."""
import numpy as np
import pytest

M64 = (1 << 64) - 1
GOLDEN = 0x9e3779b97f4a7c15
# splitmix64's first four outputs from state 0 (Vigna's published generator):
SPLITMIX0 = [0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4, 0x06c45d188009454f, 0xf88bb8a8724c81ec]


def xoshiro256p(w):
    """One step of xoshiro256+ (Blackman & Vigna): (output, next state)."""
    s0, s1, s2, s3 = w
    out = (s0 + s3) & M64
    t = (s1 << 17) & M64
    s2 ^= s0
    s3 ^= s1
    s1 ^= s2
    s0 ^= s3
    s2 ^= t
    s3 = ((s3 << 45) | (s3 >> 19)) & M64
    return out, [s0, s1, s2, s3]


def random_params(rs):
    return dict(temp=float(rs.choice([0.0, 0.5, 1.0, 1.7])), top_k=int(rs.choice([0, 1, 2, 40, 64, 511, 512, 900])),
                top_p=float(rs.choice([0.0, 0.3, 0.95, 1.0])), repeat_penalty=float(rs.choice([1.0, 1.1, 1.5])),
                repeat_last_n=int(rs.choice([0, 3, 64, 128, 5000])), freq_penalty=float(rs.choice([0.0, 0.1, 0.7])),
                presence_penalty=float(rs.choice([0.0, 0.3])), no_repeat_ngram=int(rs.choice([0, 1, 2, 3, 70])),
                seed=int(rs.integers(1 << 63)))


def random_logits(rs, nv, kind):
    lg = (rs.standard_normal(nv) * 3).astype(np.float32)
    if kind == "ties":
        lg = np.round(lg * 2) / 2                         # many exact ties
    elif kind == "zeros":
        lg = np.where(rs.random(nv) < 0.5, np.float32(0.0), np.float32(-0.0)) + np.round(lg) * (rs.random(nv) < 0.2)
        lg = lg.astype(np.float32)
    elif kind == "nan":
        lg[rs.integers(0, nv, 3)] = np.nan
    elif kind == "inf":
        lg[rs.random(nv) < 0.9] = -np.inf
    return lg.astype(np.float32)


@pytest.mark.skipif("not __import__('oracle.g4o', fromlist=['g4o']).ref_sampler_available()",
                    reason="oracle/_ref/libg4refsampler.so not built (make -C oracle ref)")
@pytest.mark.parametrize("seed", range(6))
def test_restatement_equals_reference_build(oracle, seed):
    rs = np.random.default_rng(seed)
    for trial in range(25):
        nv = int(rs.choice([1, 3, 100, 700, 5000]))
        params = random_params(rs)
        a = oracle.Sampler(nv, **params)
        b = oracle.Sampler(nv, use_ref=True, **params)
        for t in rs.integers(-2, nv + 2, size=int(rs.integers(0, 6))):
            a.ban(int(t))
            b.ban(int(t))
        # history, sometimes past the 4096-id ring so it wraps
        hist = rs.integers(0, min(nv, 8), size=int(rs.choice([0, 5, 300, 4200])))
        for t in hist:
            a.accept(int(t))
            b.accept(int(t))
        kind = ["plain", "ties", "zeros", "nan", "inf"][trial % 5]
        for step in range(12):
            lg = random_logits(rs, nv, kind)
            l1, l2 = lg.copy(), lg.copy()
            t1, t2 = a.sample(l1), b.sample(l2)
            assert t1 == t2, (trial, step, params)
            assert l1.tobytes() == l2.tobytes(), (trial, step, params)
            assert a.rng == b.rng
            a.accept(t1)
            b.accept(t2)
        assert a.recent() == b.recent()


def test_rng_seeding_is_splitmix_then_xoshiro(oracle):
    # with seed = -golden, the state is splitmix64's words from state 0
    s = oracle.Sampler(4, seed=(-GOLDEN) & M64, top_k=4, top_p=1.0)
    s.sample(np.zeros(4, np.float32))
    _, w = xoshiro256p(list(SPLITMIX0))
    assert s.rng == w
    s.sample(np.zeros(4, np.float32))
    _, w = xoshiro256p(w)
    assert s.rng == w


def test_greedy_is_first_argmax(oracle):
    rs = np.random.default_rng(3)
    for nv in (1, 7, 1000):
        s = oracle.Sampler(nv, temp=0.0)
        lg = np.round(rs.standard_normal(nv)).astype(np.float32)
        assert s.sample(lg.copy()) == int(np.argmax(lg))
        assert s.rng == [0, 0, 0, 0]                      # greedy draws no random number
    lg = np.array([np.nan, 5.0, 7.0], np.float32)        # a NaN at 0 keeps index 0
    assert oracle.Sampler(3, temp=0.0).sample(lg) == 0
    lg = np.array([1.0, np.nan, 7.0, 7.0], np.float32)   # NaNs elsewhere never win; first of a tie
    assert oracle.Sampler(4, temp=0.0).sample(lg) == 2


def test_top1_ignores_temperature_and_rng(oracle):
    rs = np.random.default_rng(4)
    for seed in range(20):
        s = oracle.Sampler(500, top_k=1, temp=3.0, seed=seed)
        lg = (rs.standard_normal(500)).astype(np.float32)
        assert s.sample(lg.copy()) == int(np.argmax(lg))


def test_bans_ngram_and_penalties_rewrite_logits(oracle):
    s = oracle.Sampler(10, temp=0.0, repeat_penalty=2.0, freq_penalty=0.5, presence_penalty=0.25, repeat_last_n=4,
                       no_repeat_ngram=2)
    s.ban(9)
    for t in (1, 2, 3, 1, 2, 2):
        s.accept(t)
    lg = np.array([0, 4, -4, 8, 1, 1, 1, 1, 1, 50], np.float32)
    s.sample(lg)
    # ban: 9; 2-gram: the newest id 2 was followed by 3 and by 2 before -> 3 and 2 banned
    assert lg[9] == -np.inf and lg[3] == -np.inf and lg[2] == -np.inf
    # window (newest 4): 2, 2, 1, 3 -> id 1 once: 4/2 - (0.5 + 0.25)
    assert lg[1] == np.float32(4 / 2 - 0.75)
    assert lg[0] == 0 and lg[4] == 1


def test_draw_frequencies_follow_the_softmax(oracle):
    # two candidates, top_p off: P(id 0) = 1 / (1 + exp(-d / temp))
    d, temp = 1.0, 0.8
    s = oracle.Sampler(2, temp=temp, top_p=1.0, seed=11)
    n, hits = 20000, 0
    for _ in range(n):
        hits += s.sample(np.array([d, 0.0], np.float32)) == 0
    p = 1.0 / (1.0 + np.exp(-d / temp))
    sd = np.sqrt(n * p * (1 - p))
    assert abs(hits - n * p) < 5 * sd


def test_top_p_keeps_the_smallest_prefix(oracle):
    # probabilities 0.5, 0.25, 0.125, ...: top_p = 0.6 keeps the first two
    nv = 8
    lg = np.array([-(i * np.log(2.0)) for i in range(nv)], np.float32)
    seen = set()
    for seed in range(200):
        s = oracle.Sampler(nv, top_p=0.6, top_k=nv, seed=seed)
        seen.add(s.sample(lg.copy()))
    assert seen == {0, 1}
