"""GPU parity of the verify-pass LM head (vnx_lm_head, matrix cores).

Reference: the fp64 product of the same bf16 inputs (x @ w.T, the tied head
of cometspark.py:396-398).  Bar: |out - ref| <= RTOL * sum_k |x_k w_k| per
element with fp32 output (fp32 accumulation of exact bf16 products: the
rounding error is a few ulps of the running sums, far below 1e-5 of the
magnitude); with bf16 output the result is additionally rounded once:
|out - ref| <= 2^-8 |ref| + RTOL * mag."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

RTOL = 1e-5


def _say(*a):
    print(*a, flush=True)


def _check(out, x, w, bf16=False):
    x64 = x.float().cpu().numpy().astype(np.float64)
    w64 = w.float().cpu().numpy().astype(np.float64)
    ref = x64 @ w64.T
    mag = np.abs(x64) @ np.abs(w64).T
    o = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(o - ref)
    tol = RTOL * mag + (2.0 ** -8 * np.abs(ref) if bf16 else 0.0)
    worst = float(np.max(err / (mag + 1e-300)))
    assert np.all(err <= tol + 1e-30), f"worst err / mag = {worst:.3e}"
    return worst


def _inputs(hip, M, K, V, seed, std_w=0.02):
    g = torch.Generator(device=hip.torch_device)
    g.manual_seed(seed)
    x = torch.randn((M, K), generator=g, device=hip.torch_device).to(torch.bfloat16)
    w = (torch.randn((V, K), generator=g, device=hip.torch_device) * std_w).to(torch.bfloat16)
    return x, w


@pytest.mark.parametrize("M,K,V", [(1, 64, 256), (17, 128, 1000), (256, 64, 4099), (100, 1024, 50000),
                                   (33, 192, 777), (224, 64, 3)])
def test_lm_head_shapes(hip, M, K, V):
    _say(f"lm_head M={M} K={K} V={V}")
    x, w = _inputs(hip, M, K, V, M + K + V)
    out = hip.lm_head(x, w)
    torch.cuda.synchronize()
    assert out.shape == (M, V) and out.dtype == torch.float32
    _say(f"  worst err / mag = {_check(out, x, w):.2e}")


def test_config5_verify_shape(hip):
    """The mate verify pass: B*(k+1) = 32*7 = 224 positions, D = 1024, the
    248,320-row tied head, written straight into a (B, k+1, V) logits buffer."""
    _say("lm_head config 5: M=224 K=1024 V=248320")
    B, k1, K, V = 32, 7, 1024, 248320
    x, w = _inputs(hip, B * k1, K, V, 5)
    logits = torch.empty((B, k1, V), dtype=torch.float32, device=hip.torch_device)
    hip.lm_head(x, w, out=logits.view(B * k1, V))
    torch.cuda.synchronize()
    _say(f"  worst err / mag = {_check(logits.view(B * k1, V), x, w):.2e}")


def test_bf16_out_and_strided_views(hip):
    _say("lm_head bf16 out, strided x")
    M, K, V = 40, 256, 10000
    x, w = _inputs(hip, M, 2 * K, V, 3)
    xs = x[:, K:]                                   # row pitch 2K
    ws = w[:, :K]                                   # row pitch 2K
    out = hip.lm_head(xs, ws, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    _check(out, xs, ws, bf16=True)
    buf = torch.full((M, V + 4), 7.0, device=hip.torch_device)
    hip.lm_head(xs, ws, out=buf[:, :V])
    torch.cuda.synchronize()
    _check(buf[:, :V], xs, ws)
    assert torch.all(buf[:, V:] == 7.0)


def test_matches_torch_bf16_matmul_closely(hip):
    """hipBLASLt's bf16 GEMM (torch.matmul) agrees to its own rounding."""
    x, w = _inputs(hip, 64, 1024, 20000, 9)
    out = hip.lm_head(x, w)
    ref = torch.matmul(x.float(), w.float().t())
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-4)


def test_rejects_bad_arguments(hip):
    dev = hip.torch_device
    x = torch.zeros((4, 96), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((10, 96), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):   # K not a multiple of 64
        hip.lm_head(x, w)
    x = torch.zeros((257, 64), dtype=torch.bfloat16, device=dev)
    w = torch.zeros((10, 64), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):   # more than 256 positions
        hip.lm_head(x, w)
