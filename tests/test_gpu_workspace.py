"""Ownership of the library's device scratch, and route choice independent of
call history.

Routes that need scratch (K-split partials of the pipelined GEMM and of the
narrow decode GEMV, dequantized weight slabs before hipBLASLt) take it from a
caller-registered stream-ordered allocator, else from a per-(device, stream)
library pool; ubridge_release_workspace frees a stream's pool buffers.  A call
first made inside a graph capture obtains its scratch and hipBLASLt plan
outside the capture, so it records the same route -- and gives the same bits
-- as an eager call.  The shapes below are used by no other test, so their
hipBLASLt plans do not exist before this module runs."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from ubridge_amd import ops, synth  # noqa: E402

pytestmark = pytest.mark.gpu


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).view(torch.bfloat16).cuda()


class _Cases:
    """One call per scratch-using route, each a closure (out, stream)."""

    def __init__(self, seed):
        g = torch.Generator().manual_seed(seed)
        self.calls = {}
        # pipelined GPTQ GEMM with K split over workgroups (8 tiles < CUs / 2)
        K, N, grp = 4096, 1544, 128
        qw, sc, qz = synth.make_gptq_w4(K, N, grp, seed=seed)
        qw, sc, qz = torch.from_numpy(qw).cuda(), _bf(sc), torch.from_numpy(qz).cuda()
        a = _bf(synth.bf16_activations(72, K, seed=seed + 1))
        self.calls["w4a16_ksplit"] = ((72, N), lambda o, s: ops.w4a16_gemm(a, qw, sc, qz, grp,
                                                                            out=o, stream=s))
        # slab route (dequantized slab + hipBLASLt) beyond 1024 tokens
        K2, N2 = 768, 1048
        qw2, sc2, qz2 = synth.make_gptq_w4(K2, N2, grp, seed=seed + 2)
        qw2, sc2, qz2 = torch.from_numpy(qw2).cuda(), _bf(sc2), torch.from_numpy(qz2).cuda()
        a2 = _bf(synth.bf16_activations(1096, K2, seed=seed + 3))
        self.calls["w4a16_slab"] = ((1096, N2), lambda o, s: ops.w4a16_gemm(a2, qw2, sc2, qz2, grp,
                                                                            out=o, stream=s))
        # narrow decode GEMV (64 column workgroups: K split, partials summed)
        K3, N3 = 8192, 1032
        qw3, sc3, qz3 = synth.make_gptq_w4(K3, N3, grp, seed=seed + 4)
        qw3, sc3, qz3 = torch.from_numpy(qw3).cuda(), _bf(sc3), torch.from_numpy(qz3).cuda()
        a3 = _bf(synth.bf16_activations(2, K3, seed=seed + 5))
        self.calls["gemv_ksplit"] = ((2, N3), lambda o, s: ops.w4a16_gemm(a3, qw3, sc3, qz3, grp,
                                                                          out=o, stream=s))
        # QMatMul at prefill size: Q4_K dequantized slab + hipBLASLt
        K4, N4 = 1024, 776
        w4 = torch.from_numpy(synth.make_weight_soa(synth.Q4_K, N4, K4, seed=seed + 6)).cuda()
        mm = ops.QMatMul(ops.Q4_K, w4, N4, K4)
        x4 = _bf(synth.bf16_activations(808, K4, seed=seed + 7))
        mm.workspace(808)
        self.calls["qmatmul_slab"] = ((808, N4), lambda o, s: mm(x4, out=o, stream=s))
        # dense matmul_bf16 above 16 tokens: hipBLASLt
        a5 = torch.randn(40, 520, generator=g).to(torch.bfloat16).cuda()
        b5 = torch.randn(520, 904, generator=g).to(torch.bfloat16).cuda()
        self.calls["dense_blaslt"] = ((1, 40, 904), lambda o, s: ops.matmul(a5, b5, out=o, stream=s))
        self.dtype = {"qmatmul_slab": torch.float32}

    def out(self, name):
        shape = self.calls[name][0]
        return torch.zeros(*shape, dtype=self.dtype.get(name, torch.bfloat16), device="cuda")


def _capture_then_eager(cases, name):
    """Capture the call on a stream whose pool was just released, replay it
    three times with eager work between, then run it eagerly: (replays,
    eager)."""
    fn = cases.calls[name][1]
    s = torch.cuda.Stream()
    ops.release_workspace(s)
    out = cases.out(name)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn(out, s)
    reps = []
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        reps.append(out.clone())
        torch.ones(1 << 20, device="cuda").sum()  # eager work between replays
    eager = cases.out(name)
    with torch.cuda.stream(s):
        fn(eager, s)
    torch.cuda.synchronize()
    del g
    ops.release_workspace(s)
    return reps, eager


@pytest.fixture(scope="module")
def cases(dev):
    return _Cases(seed=0xA11C)


@pytest.mark.parametrize("name", ["w4a16_ksplit", "w4a16_slab", "gemv_ksplit", "qmatmul_slab",
                                  "dense_blaslt"])
def test_capture_before_eager_same_bits(cases, name):
    reps, eager = _capture_then_eager(cases, name)
    assert eager.abs().sum().item() > 0
    for r in reps:
        assert torch.equal(r, eager), name


@pytest.mark.parametrize("name", ["w4a16_ksplit", "w4a16_slab", "gemv_ksplit", "qmatmul_slab"])
def test_caller_allocator(cases, name):
    # every scratch block comes from the caller's allocator and goes back to
    # it within the call; the library pool does not grow; bits equal the
    # pool route's, eager and captured
    fn = cases.calls[name][1]
    ref = cases.out(name)
    fn(ref, None)
    torch.cuda.synchronize()
    pool_before = ops.workspace_stats()[:2]
    alloc = ops.TorchWorkspaceAllocator()
    ops.set_workspace_allocator(alloc)
    try:
        out = cases.out(name)
        fn(out, None)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert alloc.calls >= 1 and not alloc.live
        assert ops.workspace_stats()[2] == 0
        s = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        out2 = cases.out(name)
        with torch.cuda.graph(g, stream=s):
            fn(out2, s)
        for _ in range(2):
            out2.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out2, ref)
        assert not alloc.live and ops.workspace_stats()[2] == 0
        del g
    finally:
        ops.set_workspace_allocator(None)
    assert ops.workspace_stats()[:2] == pool_before


def test_pool_growth_frees_outgrown_buffer(cases):
    # a stream's buffer outgrown by a larger call is freed once the work that
    # used it has finished: one live buffer per stream afterwards
    s = torch.cuda.Stream()
    ops.release_workspace(s)
    n0 = ops.workspace_stats()[0]
    for name in ("gemv_ksplit", "w4a16_ksplit", "w4a16_slab", "w4a16_ksplit"):
        out = cases.out(name)
        with torch.cuda.stream(s):
            cases.calls[name][1](out, s)
        torch.cuda.synchronize()
    assert ops.workspace_stats()[0] == n0 + 1
    ops.release_workspace(s)
    assert ops.workspace_stats()[0] == n0


def _stream_lifecycle():
    """Run in a fresh process: streams created and destroyed through the HIP
    runtime, each used by scratch-taking calls, then released."""
    # the HIP runtime torch (and so libubridge_hip) already runs on
    hip = ctypes.CDLL(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so"))
    cases = _Cases(seed=0xB0B)
    assert ops.workspace_stats() == (0, 0, 0)
    # the process's first library call is an eager decode GEMV (no hipBLASLt):
    # it makes the hipBLASLt set-up, so a dense GEMM of a new shape first met
    # inside a capture still takes hipBLASLt, as eagerly
    o = cases.out("gemv_ksplit")
    cases.calls["gemv_ksplit"][1](o, None)
    torch.cuda.synchronize()
    ops.release_workspace(None)
    reps, eager = _capture_then_eager(cases, "dense_blaslt")
    assert all(torch.equal(r, eager) for r in reps)
    refs = {}
    for name in cases.calls:
        refs[name] = cases.out(name)
        cases.calls[name][1](refs[name], None)
    torch.cuda.synchronize()
    ops.release_workspace(None)
    assert ops.workspace_stats() == (0, 0, 0)
    for rnd in range(3):
        handles = []
        for _ in range(2):
            h = ctypes.c_void_p()
            assert hip.hipStreamCreate(ctypes.byref(h)) == 0
            handles.append(h)
        for h in handles:
            st = torch.cuda.ExternalStream(h.value)
            for name in cases.calls:
                out = cases.out(name)
                with torch.cuda.stream(st):
                    cases.calls[name][1](out, st)
                torch.cuda.synchronize()
                assert torch.equal(out, refs[name]), (rnd, name)
        assert ops.workspace_stats()[0] >= 2
        for h in handles:
            ops.release_workspace(torch.cuda.ExternalStream(h.value))
            assert hip.hipStreamDestroy(h) == 0
        assert ops.workspace_stats() == (0, 0, 0), ops.workspace_stats()
    print("stream lifecycle ok")


def _init_then_capture():
    """Run in a fresh process: ubridge_init, then the first library call of
    the process is captured and equals the eager one."""
    cases = _Cases(seed=0xC0DE)
    ops.init()
    for name in ("dense_blaslt", "w4a16_slab"):
        reps, eager = _capture_then_eager(cases, name)
        assert all(torch.equal(r, eager) for r in reps), name
    print("init then capture ok")


def test_init_then_capture_first(dev):
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "init"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 0 and "init then capture ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


def test_stream_lifecycle_returns_to_zero(dev):
    r = subprocess.run([sys.executable, os.path.abspath(__file__)], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode == 0 and "stream lifecycle ok" in r.stdout, r.stdout[-2000:] + r.stderr[-4000:]


if __name__ == "__main__":
    if sys.argv[1:] == ["init"]:
        _init_then_capture()
    else:
        _stream_lifecycle()
