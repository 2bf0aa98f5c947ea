"""rie_hip_k_argmax_noalloc (the argmax entry point that allocates no device
memory: its partials live in the library's static device array) against
rie_hip_k_argmax, through the C ABI: bit-exact indices on two calls in a row,
the second with a smaller input, the same on a caller's stream and recorded in a
captured graph, and a clear error past the array's limit."""
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
    rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), x.size, b.data_ptr(), None, err, 256)
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
        rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), n, out.data_ptr(), None, err, 256)
        assert rc == -5 and b"outside 1..1048576" in err.value, (n, rc, err.value)


def test_argmax_noalloc_on_a_stream_and_under_graph_capture():
    """On the caller's stream the call only queues its kernels; recorded in a
    captured graph (where nothing may allocate), every replay over new input
    values gives the allocating argmax's index for those values."""
    assert torch.cuda.is_available(), "needs the MI355X"
    cuda = torch.device("cuda:0")
    L = R.lib()
    rng = np.random.default_rng(12)
    n = 151936
    err = C.create_string_buffer(256)
    xd = torch.zeros(n, dtype=torch.float32, device=cuda)
    out = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    ref = torch.full((1,), -1, dtype=torch.int32, device=cuda)
    # a plain call on a side stream first (it also looks up the array's address)
    side = torch.cuda.Stream()
    x = rng.standard_normal(n).astype(np.float32)
    xd.copy_(torch.from_numpy(x))
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), n, out.data_ptr(), C.c_void_p(side.cuda_stream), err, 256)
    assert rc == 0, err.value
    side.synchronize()
    assert int(out.cpu()[0]) == int(np.argmax(x))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream().cuda_stream
        rc = L.rie_hip_k_argmax_noalloc(xd.data_ptr(), n, out.data_ptr(), C.c_void_p(st), err, 256)
    assert rc == 0, err.value
    for rep in range(4):
        x = rng.standard_normal(n).astype(np.float32)
        x[(rep * 7919) % n] = x[n - 1 - rep] = x.max() + 1.0  # a tie: the first index wins
        xd.copy_(torch.from_numpy(x))
        out.fill_(-1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert L.rie_hip_k_argmax(xd.data_ptr(), n, ref.data_ptr()) == 0
        want = min((rep * 7919) % n, n - 1 - rep)
        assert int(out.cpu()[0]) == int(ref.cpu()[0]) == want, rep
