"""GPU checks of the achievable-peak probes bench.py reports beside the
datasheet peaks (peak_probe.hip): the read probe touches every 16-byte chunk
exactly once (the XOR of its per-workgroup words equals the XOR of the
buffer), and the MFMA probe's output is finite and repeatable."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n_words,n_wg", [(4, 1), (4096, 3), (1 << 20, 64), ((1 << 20) + 12, 257)])
def test_probe_read_covers_buffer_once(gpu, n_words, n_wg):
    la = gpu
    rng = np.random.default_rng(n_words)
    data = rng.integers(0, 2**32, n_words, dtype=np.uint64).astype(np.uint32)
    src = la.DeviceArray.from_numpy(data)
    sink = la.DeviceArray.zeros(n_wg, np.uint32)
    assert la.load().lfm_hip_probe_read(src.ptr, n_words * 4, sink.ptr, n_wg, None) == 0
    want = np.bitwise_xor.reduce(data[: (n_words * 4 // 16) * 4])
    assert np.bitwise_xor.reduce(sink.numpy()) == want


def test_probe_mfma_repeatable(gpu):
    la = gpu
    out = la.DeviceArray.zeros(8 * 256, np.float32)
    assert la.load().lfm_hip_probe_mfma(out.ptr, 8, 16, None) == 0
    a = out.numpy().copy()
    assert la.load().lfm_hip_probe_mfma(out.ptr, 8, 16, None) == 0
    assert np.all(np.isfinite(a)) and np.array_equal(a, out.numpy()) and np.any(a != 0)
