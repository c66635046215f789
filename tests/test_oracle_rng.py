"""The oracle's RNG against rng.rs's own known answers and invariants (rng.rs:64-144)."""
from oracle_lib import Rng


def test_a_seed_gives_the_same_numbers_everywhere():
    # rng.rs:71-86: the first three outputs for seeds 0 and 1.
    def first(seed):
        r = Rng(seed)
        return [r.next_u64(), r.next_u64(), r.next_u64()]

    assert first(0) == [0x99EC5F36CB75F2B4, 0xBF6E1F784956452A, 0x1A5F849D4933E6E0]
    assert first(1) == [0xB3F2AF6D0FC710C5, 0x853B559647364CEA, 0x92F89756082A4514]


def _splitmix_xoshiro_python(seed, n):
    # An independent restatement from the published algorithms (Blackman and Vigna).
    M = (1 << 64) - 1
    x = seed
    s = []
    for _ in range(4):
        x = (x + 0x9E3779B97F4A7C15) & M
        z = x
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        s.append(z ^ (z >> 31))
    rotl = lambda v, k: ((v << k) | (v >> (64 - k))) & M
    out = []
    for _ in range(n):
        out.append((rotl((s[1] * 5) & M, 7) * 9) & M)
        t = (s[1] << 17) & M
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = rotl(s[3], 45)
    return out


def test_the_stream_matches_an_independent_restatement():
    for seed in [0, 1, 2, 1234, 1235, 2**63 + 5, 2**64 - 1]:
        r = Rng(seed)
        assert [r.next_u64() for _ in range(50)] == _splitmix_xoshiro_python(seed, 50), seed


def test_below_covers_every_value_and_never_reaches_n():
    r = Rng(7)
    seen = [0] * 7
    for _ in range(7000):
        seen[r.below(7)] += 1
    assert all(850 <= c < 1150 for c in seen), seen
    assert r.below(1) == 0


def test_unit_stays_in_the_half_open_interval():
    r = Rng(3)
    total = 0.0
    for _ in range(10000):
        u = r.unit()
        assert 0.0 <= u < 1.0
        total += u
    assert abs(total / 10000 - 0.5) < 0.01


def test_unit_is_the_top_53_bits():
    a, b = Rng(99), Rng(99)
    for _ in range(100):
        assert a.unit() == (b.next_u64() >> 11) * 2.0**-53


def test_below_redraws_for_a_huge_n():
    # rng.rs:117-138: n = 2^63 + 1, about half the draws are redrawn.
    n = (1 << 63) + 1
    a, b = Rng(11), Rng(11)
    M = (1 << 64) - 1
    redraws = 0
    for _ in range(200):
        m = b.next_u64() * n
        if (m & M) < n:
            floor = ((-n) & M) % n
            while (m & M) < floor:
                redraws += 1
                m = b.next_u64() * n
        got = a.below(n)
        assert got < n
        assert got == m >> 64
    assert redraws > 0
