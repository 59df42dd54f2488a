"""GPU parity of lfm_hip_fnv1a64 (the parallel FNV-1a 64 the .lfmcache
writer and loader use for their checksum) against the oracle's sequential
FNV-1a (orc_fnv1a, pinned to the published FNV test vectors in
test_cache_oracle.py).  Bit-exact: the hash is integer arithmetic mod 2^64."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BASIS = 14695981039346656037


@pytest.mark.parametrize("n", [1, 15, 16, 17, 1023, 1024, 1025, 4096 + 3, 64 * 1024, 64 * 1024 + 1,
                               64 * 64 * 1024 + 5, 10_000_019])
def test_fnv1a64_matches_oracle(gpu, orc, n):
    la = gpu
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, n, dtype=np.uint8)
    d = la.DeviceArray.from_numpy(data)
    assert la.fnv1a64(d, n) == orc.fnv1a(data)
    h_in = int(rng.integers(0, 2**63)) * 2 + 1
    assert la.fnv1a64(d, n, h_in) == orc.fnv1a(data, h_in)


def test_fnv1a64_published_vectors_and_edges(gpu):
    la = gpu
    for text, want in ((b"a", 0xAF63DC4C8601EC8C), (b"foobar", 0x85944171F73967E8)):
        d = la.DeviceArray.from_numpy(np.frombuffer(text, np.uint8).copy())
        assert la.fnv1a64(d, len(text)) == want
    assert la.fnv1a64(None, 0) == BASIS
    z = la.DeviceArray.from_numpy(np.zeros(300_000, np.uint8))
    ff = la.DeviceArray.from_numpy(np.full(300_000, 255, np.uint8))
    hz, hf = la.fnv1a64(z, 300_000), la.fnv1a64(ff, 300_000)
    from oracle.bindings import Oracle
    o = Oracle()
    assert hz == o.fnv1a(np.zeros(300_000, np.uint8)) and hf == o.fnv1a(np.full(300_000, 255, np.uint8))
    with pytest.raises(la.LfmAttnError):
        la.fnv1a64(int(z) + 1, 16)  # the device buffer must be 16-byte aligned
