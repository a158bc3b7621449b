"""qwen_hip_linear_nobias_bf16_noalloc (the op-level linear that allocates
nothing: its temporary memory is a fixed per-GPU device array) against
qwen_hip_linear_nobias_bf16 (the same product on the library's grown
workspace), through the C ABI.  Both run the same kernels with the same
tiling, so the results must be identical bit for bit; two calls in a row,
the second one smaller, show that the shared array's leftover contents from
the first call do not leak into the second."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(qa, torch, S, K, N, seed):
    lib = qa.lib()
    W = qa.synth_bf16(N * K, 0, 9500 + seed).reshape(N, K)
    x = qa.synth_f32(S * K, 0, 9600 + seed).reshape(S, K)
    dW = torch.from_numpy(W.view(np.int16)).cuda()
    dx = torch.from_numpy(x).cuda()
    y_ref = torch.full((S, N), float("nan"), dtype=torch.float32, device="cuda")
    y_na = torch.full((S, N), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    qa.check(lib.qwen_hip_linear_nobias_bf16(y_ref.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, K, N, None),
             "linear")
    qa.check(lib.qwen_hip_linear_nobias_bf16_noalloc(y_na.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, K, N, None),
             "linear_noalloc")
    torch.cuda.synchronize()
    a, b = y_ref.cpu().numpy(), y_na.cpu().numpy()
    assert np.isfinite(a).all()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), float(np.abs(a - b).max())
    # and against an fp64 product of the same operands (the op's accuracy bar)
    ref = x.astype(np.float64) @ qa.bf16_to_f32(W).astype(np.float64).T
    bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(qa.bf16_to_f32(W)).astype(np.float64).T) + 1e-6
    assert (np.abs(b - ref) <= bound).all()


def test_noalloc_matches_linear_twice(qa, gpu):
    torch = gpu
    # a split-K product (small tile grid) first, then a smaller one: the second
    # reads only what it wrote over the first one's leftovers
    _case(qa, torch, 300, 1024, 2048, 1)
    _case(qa, torch, 40, 1024, 1024, 2)
    _case(qa, torch, 1, 1024, 3072, 3)      # seq 1: the GEMV, no scratch at all


def test_noalloc_above_512_rows(qa, gpu):
    """More than 512 rows: 128 x 128 tiles.  1024 x 1024 -> 4096 has 256 output
    tiles, enough to fill the chip, so the op keeps one split and needs only
    the 4 MiB of x halves; then a smaller product over the leftovers."""
    torch = gpu
    _case(qa, torch, 1024, 1024, 4096, 4)
    _case(qa, torch, 600, 1024, 1024, 5)    # 5 x 8 tiles: split K, partials in the array


CAPTURE = r"""
import importlib, sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
qa = importlib.import_module("qwen-asr_amd")
lib = qa.lib()
S, K, N = 96, 1024, 2048
W = qa.synth_bf16(N * K, 0, 9700).reshape(N, K)
x = qa.synth_f32(S * K, 0, 9701).reshape(S, K)
dW = torch.from_numpy(W.view(np.int16)).cuda()
dx = torch.from_numpy(x).cuda()
y_ref = torch.empty((S, N), dtype=torch.float32, device="cuda")
y = torch.full((S, N), float("nan"), dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
qa.check(lib.qwen_hip_linear_nobias_bf16(y_ref.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, K, N, None), "linear")
torch.cuda.synchronize()
ref = y_ref.cpu().numpy().view(np.uint32)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    # the process's first no-alloc call: it looks up the array's address here
    rc = lib.qwen_hip_linear_nobias_bf16_noalloc(y.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, K, N,
                                                 torch.cuda.current_stream().cuda_stream)
assert rc == 0, (rc, qa.last_error())
for i in range(3):
    y.fill_(float("nan"))
    z = (dx * 2.0).sum()                 # eager work between the replays
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, ref), f"replay {i}: results differ"
print("capture ok: 3 replays equal the eager product bit for bit", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture(qa, gpu):
    """A fresh process whose first no-alloc call happens while a HIP graph is
    being captured (torch.cuda.graph): the capture succeeds, and each of three
    replays, with eager work between them, writes the eager op's result bit
    for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", CAPTURE, root], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "capture ok" in r.stdout


def test_noalloc_rejects_oversize(qa, gpu):
    torch = gpu
    lib = qa.lib()
    cap = lib.qwen_hip_linear_noalloc_max_bytes()
    assert cap == 32 << 20
    S, K, N = 8192, 2048, 128                # 4 * S * K = 64 MiB of hi/lo split > 32 MiB
    dW = torch.zeros((N, K), dtype=torch.int16, device="cuda")
    dx = torch.zeros((S, K), dtype=torch.float32, device="cuda")
    dy = torch.zeros((S, N), dtype=torch.float32, device="cuda")
    rc = lib.qwen_hip_linear_nobias_bf16_noalloc(dy.data_ptr(), dx.data_ptr(), dW.data_ptr(), S, K, N, None)
    assert rc == -1, rc
    assert "scratch" in qa.last_error()
