"""rie_hip_k_argmax_noalloc (the argmax entry point that allocates no device
memory: its partials live in the library's static device array) against
rie_hip_k_argmax, through the C ABI: bit-exact indices on two calls in a row,
the second with a smaller input, and a clear error past the array's limit."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

import rust_interference_engine_amd as R  # noqa: E402


def _both(L, x, cuda):
    xd = torch.from_numpy(x).to(cuda)
    a = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    b = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    assert L.rie_hip_k_argmax(xd.data_ptr(), x.size, a.data_ptr()) == 0
    err = C.create_string_buffer(256)
    rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), x.size, b.data_ptr(), err, 256)
    assert rc == 0, err.value
    return int(a.cpu()[0]), int(b.cpu()[0])


def test_argmax_noalloc_equals_allocating_argmax():
    assert torch.cuda.is_available(), "needs the MI355X"
    cuda = torch.device("cuda:0")
    L = R.lib()
    rng = np.random.default_rng(11)
    # two calls in a row, the second smaller: the array keeps the first call's
    # partials, which the second must neither read nor depend on
    for n in (1048576, 151936, 128256, 4099, 1000, 1):
        x = rng.standard_normal(n).astype(np.float32)
        if n > 8:
            x[n // 5] = x[n - 3] = x.max() + 2.0  # tie: the first index wins
        want = n // 5 if n > 8 else int(np.argmax(x))
        a, b = _both(L, x, cuda)
        assert a == b == want, (n, a, b, want)
    # the same input twice: same answer, nothing carried between calls
    x = rng.standard_normal(70000).astype(np.float32)
    assert _both(L, x, cuda) == _both(L, x, cuda) == (int(np.argmax(x)),) * 2


def test_argmax_noalloc_rejects_sizes_past_its_array():
    assert torch.cuda.is_available(), "needs the MI355X"
    cuda = torch.device("cuda:0")
    L = R.lib()
    xd = torch.zeros(8, dtype=torch.float32, device=cuda)
    out = torch.zeros(1, dtype=torch.int32, device=cuda)
    err = C.create_string_buffer(256)
    for n in (1048577, 0):  # nothing is launched for these: the host rejects them first
        rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), n, out.data_ptr(), err, 256)
        assert rc == -5 and b"outside 1..1048576" in err.value, (n, rc, err.value)
