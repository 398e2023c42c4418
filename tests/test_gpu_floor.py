"""The measurement-only stream floor (nis_stream_floor): the sparse kernel's
row layout and load pipeline computing each row's max and sum of
2^(x c - ceil(max c)).  bench.py --floor times it as the bandwidth ceiling
of the sparse kernel; this checks that it reads every element of every row
(the max exactly, the sum against an f64 reference within f32 accuracy).
The split floor (nis_stream_floor_split, bench.py --floor --split S) reads
each row in S slices and merges their partials in a second launch; it must
give the same results."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("V,ld", [(50257, 50257), (50257, 50261), (256, 259), (4100, 4100),
                                  (53245, 53248)])
def test_floor_reads_every_element(V, ld):
    import torch
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(V + ld))
    B = 40
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    # the max planted at the first, last and a middle element of some rows
    for r, j in ((0, 0), (1, V - 1), (2, V // 2), (3, 1), (4, V - 2)):
        x[r, j] = np.float32(30.0)
    buf = torch.full((B, ld), float("nan"), dtype=torch.float32, device="cuda:0")
    buf[:, :V] = torch.from_numpy(x).cuda()
    s = ns.Sampler(0)
    T = 0.8
    out = s.stream_floor(buf, T, V=V)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    c = np.float64(np.float32(1.4426950408889634 / np.float64(np.float32(T))))
    M = x.max(axis=1)
    assert np.array_equal(got[:, 0], M.astype(np.float64))
    R = np.ceil(np.float32(M * np.float32(c))).astype(np.float64)
    z = np.exp2(x.astype(np.float64) * c - R[:, None]).sum(axis=1)
    assert (np.abs(got[:, 1] - z) / z).max() < 2e-6
    s.close()


def test_floor_rejects_bad_arguments():
    import ctypes
    import torch
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    x = torch.zeros((2, 300), dtype=torch.float32, device="cuda:0")
    o = torch.zeros((2, 2), dtype=torch.float32, device="cuda:0")
    L = ns.load_library()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    assert L.nis_stream_floor(s._ctx, p(x), 300, 2, 100, 1.0, p(o)) == ns.NIS_EINVAL   # V < 256
    assert L.nis_stream_floor(s._ctx, p(x), 299, 2, 300, 1.0, p(o)) == ns.NIS_EINVAL   # ld < V
    assert L.nis_stream_floor(s._ctx, p(x), 300, 2, 300, 0.0, p(o)) == ns.NIS_EINVAL   # T <= 0
    assert L.nis_stream_floor(s._ctx, None, 300, 2, 300, 1.0, p(o)) == ns.NIS_EINVAL
    s.close()


@pytest.mark.parametrize("V,ld,S", [(50257, 50257, 16), (50257, 50261, 4), (256, 259, 1),
                                    (256, 259, 3), (4100, 4100, 64), (53245, 53248, 7)])
def test_split_floor_matches_the_floor(V, ld, S):
    # nis_stream_floor_split: the same max exactly and the same sum within
    # f32 accuracy, whatever the number of slices (misaligned rows included)
    import torch
    import nimbus_sampler as ns
    rnd = np.random.Generator(np.random.PCG64(V + ld + S))
    B = 24
    x = (rnd.standard_normal((B, V)) * 3.0).astype(np.float32)
    for r, j in ((0, 0), (1, V - 1), (2, V // 2), (3, 1), (4, V - 2)):
        x[r, j] = np.float32(30.0)
    buf = torch.full((B, ld), float("nan"), dtype=torch.float32, device="cuda:0")
    buf[:, :V] = torch.from_numpy(x).cuda()
    s = ns.Sampler(0)
    T = 0.8
    print(f"[split floor] V={V} ld={ld} S={S}", flush=True)
    out = s.stream_floor_split(buf, T, S, V=V)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    c = np.float64(np.float32(1.4426950408889634 / np.float64(np.float32(T))))
    M = x.max(axis=1)
    assert np.array_equal(got[:, 0], M.astype(np.float64))
    R = np.ceil(np.float32(M * np.float32(c))).astype(np.float64)
    z = np.exp2(x.astype(np.float64) * c - R[:, None]).sum(axis=1)
    assert (np.abs(got[:, 1] - z) / z).max() < 2e-6
    s.close()


def test_split_floor_rejects_bad_arguments():
    import ctypes
    import torch
    import nimbus_sampler as ns
    s = ns.Sampler(0)
    x = torch.zeros((2, 50257), dtype=torch.float32, device="cuda:0")
    o = torch.zeros((2, 2), dtype=torch.float32, device="cuda:0")
    part = torch.zeros((2 * 64 * 4, 4), dtype=torch.float32, device="cuda:0")
    L = ns.load_library()
    p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    f = L.nis_stream_floor_split
    assert f(s._ctx, p(x), 50257, 2, 50257, 1.0, 0, p(part), p(o)) == ns.NIS_EINVAL   # S < 1
    assert f(s._ctx, p(x), 50257, 2, 50257, 1.0, 65, p(part), p(o)) == ns.NIS_EINVAL  # S > 64
    assert f(s._ctx, p(x), 50257, 2, 50257, 1.0, 3, p(part), p(o)) == ns.NIS_EINVAL   # slices > 4096 slots
    assert f(s._ctx, p(x), 50257, 2, 50257, 1.0, 4, None, p(o)) == ns.NIS_EINVAL
    assert f(s._ctx, p(x), 50257, 2, 50257, 0.0, 4, p(part), p(o)) == ns.NIS_EINVAL   # T <= 0
    s.close()
