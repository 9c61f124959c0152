"""CPU: the C form of the synthetic SplitMix64 stream (libhp_synth.so,
threaded) against its numpy definition, over sizes below and above the
one-thread threshold (2^20 words), thread counts that split the range
unevenly, and starts near 2^64 where the counter wraps."""
import numpy as np
import pytest

from heliopause_amd import synthetic as S

CASES = [  # (seed, start, n, threads)
    (1, 0, 4096, 16),
    (0x9E3779B97F4A7C15, 12345, 5001, 3),
    (7, 0, (1 << 20) - 1, 16),
    (7, 0, (1 << 20) + 12345, 16),
    (2**64 - 1, 99, (1 << 20) + 7, 3),
    (5, 2**63, 70001, 5),
    (5, 2**64 - 10, 9000, 1),                 # the counter wraps past 2^64
    (11, 2**64 - 600000, (1 << 20) + 3, 7),   # ... inside a threaded draw
]


@pytest.fixture(scope="module")
def synth():
    L = S._synth_lib()
    if L is None:
        pytest.skip("libhp_synth.so is not built (heliopause_amd.build.build_synth)")
    return L


@pytest.mark.parametrize("seed,start,n,threads", CASES)
def test_c_stream_matches_numpy(synth, seed, start, n, threads):
    got = S.splitmix64(seed, n, start, threads=threads)
    ref = S.splitmix64_numpy(seed, n, start)
    assert got.dtype == np.uint64 and got.shape == (n,)
    assert np.array_equal(got, ref)


def test_known_words():
    """The first draws of stream 0: SplitMix64's published sequence for seed
    0 (state advanced by the golden gamma before each mix)."""
    w = S.splitmix64_numpy(0, 3)
    assert [int(v) for v in w] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_split_is_contiguous():
    """Two draws of adjacent ranges give the draw of their union."""
    a = S.splitmix64(3, 300000, 2**64 - 100000)
    b = S.splitmix64(3, 5000, 2**64 - 100000 + 300000 - 2**64)
    whole = S.splitmix64(3, 305000, 2**64 - 100000)
    assert np.array_equal(np.concatenate([a, b]), whole)
