"""GPU test of dels_lowrank_argmax_noalloc, the draft step whose workspace is a
device array of the library instead of caller memory.

Called through the C ABI (ctypes) and compared, bit for bit, with
dels_lowrank_argmax on a fresh zeroed workspace: same kernels, so the same ids
and scores.  Each case makes two calls in a row, the second with a smaller
input, so the second runs on what the first left in the shared array.  The
first test checks, in a fresh child process (so that no earlier call has set
the array up), that a first call under stream capture is refused, since that
call clears the array.
"""

import os
import subprocess
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

DELS_OK, DELS_ERR_INVALID_ARGUMENT, DELS_ERR_WORKSPACE = 0, -1, -4


def _inputs(pkg, dev, M, d, r, V, seed, packed, base_dtype=torch.float32):
    x = pkg.synth.lowrank_inputs(M, d, r, V, seed=seed, base_dtype=base_dtype, act="silu").to(dev)
    A, B = (pkg.pack_operand(x.A), pkg.pack_operand(x.B)) if packed else (x.A, x.B)
    return x, A, B


def _args(pkg, x, A, B, out_ids, out_score):
    """Arguments of dels_lowrank_argmax up to ld_out (as ops.lowrank_argmax passes them)."""
    ops = pkg.ops
    M, d = x.h.shape
    a_ptr, lda, a_lay, r, _ = ops._weight(A, "A", cols=d)
    b_ptr, ldb, b_lay, V, _ = ops._weight(B, "B", cols=r)
    return [x.h.data_ptr(), x.h.stride(0), a_ptr, lda, a_lay, None, pkg._lib.ACT_SILU, b_ptr, ldb, b_lay,
            x.base.data_ptr(), x.base.stride(0), ops._DTYPES[x.base.dtype], x.prior.data_ptr(),
            ops._DTYPES[x.prior.dtype], x.alpha.data_ptr(), 1, x.beta.data_ptr(), 1, M, d, r, V,
            out_ids.data_ptr(), out_score.data_ptr(), 1]


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(pkg, x, A, B):
    lib = pkg._lib.load()
    M, d = x.h.shape
    r, V = x.A.shape[0], x.B.shape[0]
    ids = torch.full((M,), -7, dtype=torch.int64, device=x.h.device)
    sc = torch.full((M,), -7.0, dtype=torch.float32, device=x.h.device)
    ws = pkg.ops.new_workspace(x.h.device, lib.dels_lowrank_argmax_ws_bytes(M, d, r, V))
    rc = lib.dels_lowrank_argmax(*_args(pkg, x, A, B, ids, sc), ws.data_ptr(), ws.numel(), _stream())
    assert rc == DELS_OK, lib.dels_last_error()
    return ids, sc


def _noalloc(pkg, x, A, B):
    lib = pkg._lib.load()
    M = x.h.shape[0]
    ids = torch.full((M,), -7, dtype=torch.int64, device=x.h.device)
    sc = torch.full((M,), -7.0, dtype=torch.float32, device=x.h.device)
    rc = lib.dels_lowrank_argmax_noalloc(*_args(pkg, x, A, B, ids, sc), _stream())
    assert rc == DELS_OK, lib.dels_last_error()
    return ids, sc


_FIRST_CALL_CHILD = r"""
import sys
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[2])
import torch
import __graft_entry__
import test_zz_no_alloc as t
pkg = __graft_entry__.load_package()
dev = torch.device("cuda:0")
lib = pkg._lib.load()
x, A, B = t._inputs(pkg, dev, 4, 256, 64, 3001, seed=1, packed=True)
ids = torch.zeros(4, dtype=torch.int64, device=dev)
sc = torch.zeros(4, dtype=torch.float32, device=dev)
torch.cuda.synchronize()
side = torch.cuda.Stream()
graph = torch.cuda.CUDAGraph()
with torch.cuda.stream(side):
    with torch.cuda.graph(graph, stream=side):
        rc = lib.dels_lowrank_argmax_noalloc(*t._args(pkg, x, A, B, ids, sc), side.cuda_stream)
assert rc == t.DELS_ERR_INVALID_ARGUMENT, rc
assert b"must not be captured" in lib.dels_last_error()
del graph
# after the refusal an eager call sets the array up and matches the workspace entry point
got = t._noalloc(pkg, x, A, B)
want = t._with_workspace(pkg, x, A, B)
torch.cuda.synchronize()
assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])
print("first-call child ok", flush=True)
"""


def test_first_call_under_capture_is_refused():
    """In a child process that has made no call of the entry point yet."""
    print("case noalloc: first call under capture (child process)", flush=True)
    here = os.path.dirname(os.path.abspath(__file__))
    res = subprocess.run([sys.executable, "-c", _FIRST_CALL_CHILD, os.path.dirname(here), here],
                         capture_output=True, text=True, timeout=110)
    assert res.returncode == 0 and "first-call child ok" in res.stdout, (res.returncode, res.stdout[-2000:],
                                                                         res.stderr[-2000:])


@pytest.mark.parametrize("first,second", [
    # the one-launch decode step (packed weights, M <= 16): Qwen3-8B shape, then a smaller one
    ((16, 4096, 512, 151936, True), (5, 1024, 128, 20011, True)),
    # rank GEMM + MFMA-tiled argmax (M >= 64), then rank GEMM + GEMV argmax with row-major weights
    ((512, 4096, 512, 151936, True), (40, 2560, 256, 30000, False)),
])
def test_noalloc_matches_workspace_entry_point(pkg, dev, first, second):
    for i, (M, d, r, V, packed) in enumerate((first, second)):
        print(f"case noalloc call {i}: M={M} d={d} r={r} V={V} packed={packed}", flush=True)
        x, A, B = _inputs(pkg, dev, M, d, r, V, seed=M + d + i, packed=packed,
                          base_dtype=torch.bfloat16 if M >= 64 else torch.float32)
        want = _with_workspace(pkg, x, A, B)
        got = _noalloc(pkg, x, A, B)
        torch.cuda.synchronize()
        assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_oversized_shape_is_refused(pkg, dev):
    print("case noalloc: oversized shape", flush=True)
    lib = pkg._lib.load()
    need = lib.dels_lowrank_argmax_ws_bytes(1024, 4096, 512, 151936)
    assert need > pkg._lib.NOALLOC_SCRATCH_BYTES
    x, A, B = _inputs(pkg, dev, 4, 256, 64, 3001, seed=2, packed=True)
    ids = torch.zeros(4, dtype=torch.int64, device=dev)
    sc = torch.zeros(4, dtype=torch.float32, device=dev)
    args = _args(pkg, x, A, B, ids, sc)
    args[19:23] = [1024, 4096, 512, 151936]           # M, d, r, V: checked before anything runs
    rc = lib.dels_lowrank_argmax_noalloc(*args, _stream())
    assert rc == DELS_ERR_WORKSPACE and b"scratch" in lib.dels_last_error()


def test_captured_noalloc_replays(pkg, dev):
    """After the first call, the entry point may be captured: every replay, with eager
    calls of other shapes on the same array in between, reproduces the eager result."""
    print("case noalloc: captured replays", flush=True)
    x, A, B = _inputs(pkg, dev, 16, 2048, 256, 50021, seed=5, packed=True)
    y, Ay, By = _inputs(pkg, dev, 9, 1024, 128, 20011, seed=6, packed=True)
    want = _noalloc(pkg, x, A, B)
    want = (want[0].clone(), want[1].clone())
    lib = pkg._lib.load()
    ids = torch.zeros(16, dtype=torch.int64, device=dev)
    sc = torch.zeros(16, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            rc = lib.dels_lowrank_argmax_noalloc(*_args(pkg, x, A, B, ids, sc), side.cuda_stream)
    assert rc == DELS_OK, lib.dels_last_error()
    torch.cuda.synchronize()
    for _ in range(3):
        ids.fill_(-1)
        sc.fill_(0.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ids, want[0]) and torch.equal(sc, want[1])
        _noalloc(pkg, y, Ay, By)                       # another shape on the same array in between
        torch.cuda.synchronize()
