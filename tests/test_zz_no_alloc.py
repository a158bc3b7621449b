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
