"""Dense decoder-layer ops on the device (mi_linear, mi_rms_norm_residual,
mi_silu_mul via microinfer_amd.layer.hip_dense) against float32 torch
references of the same math, at the engine's decode shapes.

Projections: every Qwen3-0.6B / 8B projection shape at 1..64 rows and each
workgroup shape the launcher picks (4 or 8 waves, 16 or 32 columns); results
are reproducible bit for bit, and a captured graph gives the eager result on
every replay. RMSNorm: the residual sum is torch's bf16 addition
bit for bit and the normalised rows are within one rounding of torch's
rms_norm; SwiGLU: within one rounding of F.silu(gate) * up.
"""

import pytest
import torch
import torch.nn.functional as F

from microinfer_amd.layer.hip_dense import (hip_linear, hip_linear_swiglu, hip_rms_norm_residual,
                                            hip_silu_mul)
from microinfer_amd.runner import capture_graph

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")

# (n, k): QKV, output, gate/up and down projections of Qwen3-0.6B and 8B,
# the 0.6B vocabulary projection, and a small shape with a partial
# 64-column block.
SHAPES = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072), (6144, 4096),
          (4096, 4096), (24576, 4096), (4096, 12288), (151936, 1024), (48, 64)]


def _ulps(a, b):
    """Largest distance in units of the last place between two 16-bit
    tensors (sign-magnitude bits mapped to a monotone integer line)."""
    def line(t):
        bits = t.view(torch.int16).int()
        return torch.where(bits < 0, -(bits & 0x7FFF), bits)
    return int((line(a) - line(b)).abs().max())


def _reference(x, w):
    return (x.float() @ w.float().t())


def _assert_close(y, ref):
    # One rounding of the float32 sum to the 16-bit type, plus float32
    # summation-order differences far below it.
    err = (y.float() - ref).abs()
    tol = 8e-3 * ref.abs() + 1e-3 * ref.abs().max() + 1e-6
    assert bool((err <= tol).all()), float((err - tol).max())


@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [1, 7, 16, 33, 64])
def test_linear_matches_float32(m, n, k):
    torch.manual_seed(m * 1000 + n + k)
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    w = (0.05 * torch.randn(n, k, device=DEV)).to(torch.bfloat16)
    y = hip_linear(x, w)
    _assert_close(y, _reference(x, w))
    assert torch.equal(hip_linear(x, w), y)  # reproducible


@pytest.mark.parametrize("m,n,k", [(2, 32768, 64), (2, 32768, 96), (2, 4096, 64), (16, 4096, 416),
                                   (20, 8192, 96), (40, 2048, 160), (64, 6144, 224)])
def test_linear_partial_chunks(m, n, k):
    """k ranges that leave a wave a partial chunk of k-steps (or none), under
    every workgroup shape the launcher picks (4 or 8 waves, 16 or 32
    columns, row-tiled or not)."""
    torch.manual_seed(m + n + k)
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    w = (0.05 * torch.randn(n, k, device=DEV)).to(torch.bfloat16)
    y = hip_linear(x, w)
    assert not bool(torch.isnan(y).any())
    _assert_close(y, _reference(x, w))


def test_linear_f16_and_strided_rows():
    torch.manual_seed(3)
    m, n, k = 40, 1024, 3072
    base = torch.randn(m, k + 64, device=DEV).to(torch.float16)
    x = base[:, 32:32 + k]  # row stride k + 64, 64-byte offset
    w = (0.05 * torch.randn(n, k, device=DEV)).to(torch.float16)
    out = torch.empty(m, n + 16, device=DEV, dtype=torch.float16)[:, :n]
    y = hip_linear(x, w, out=out)
    assert y.data_ptr() == out.data_ptr()
    _assert_close(y, _reference(x, w))


def test_linear_rejects_what_it_cannot_take():
    w = torch.randn(1024, 3072, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        hip_linear(torch.randn(65, 3072, device=DEV).to(torch.bfloat16), w)
    with pytest.raises(ValueError):
        hip_linear(torch.randn(8, 3072, device=DEV), w.float())
    with pytest.raises(ValueError):
        hip_linear(torch.randn(8, 3072, device=DEV).to(torch.bfloat16), w[:1000])


def test_linear_graph_replays_match_eager():
    torch.manual_seed(5)
    m = 64
    shapes = [(4096, 1024), (1024, 2048), (6144, 1024), (1024, 3072)]
    xs = [torch.randn(m, k, device=DEV).to(torch.bfloat16) for _, k in shapes]
    ws_w = [(0.05 * torch.randn(n, k, device=DEV)).to(torch.bfloat16) for n, k in shapes]
    outs = [torch.empty(m, n, device=DEV, dtype=torch.bfloat16) for n, _ in shapes]

    def run():
        for x, w, o in zip(xs, ws_w, outs):
            hip_linear(x, w, out=o)

    run()
    eager = [o.clone() for o in outs]
    for x, w, e in zip(xs, ws_w, eager):
        _assert_close(e, _reference(x, w))
    graph = torch.cuda.CUDAGraph()
    with capture_graph(graph):
        run()
    for replay in range(4):
        for o in outs:
            o.fill_(7.0)
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), replay
        run()  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,dim", [(1, 1024), (64, 1024), (37, 4096), (5, 8192), (3, 520)])
def test_rms_norm_residual_matches_torch(dtype, rows, dim):
    torch.manual_seed(rows + dim)
    x = torch.randn(rows, dim, device=DEV).to(dtype)
    r = torch.randn(rows, dim, device=DEV).to(dtype)
    w = (1 + 0.1 * torch.randn(dim, device=DEV)).to(dtype)
    out, combined = hip_rms_norm_residual(x, r, w, 1e-6)
    want_sum = x + r
    assert torch.equal(combined, want_sum)
    ref = F.rms_norm(want_sum.float(), (dim,), w.float(), 1e-6)
    err = (out.float() - ref).abs()
    assert bool((err <= 1.6e-2 * ref.abs() + 1e-6).all())
    # Against torch's own 16-bit rms_norm: equal or one unit apart.
    torch_out = F.rms_norm(want_sum, (dim,), w, 1e-6)
    assert _ulps(out, torch_out) <= 1
    # No residual: the sum is x itself.
    out0, same = hip_rms_norm_residual(x, None, w, 1e-6)
    assert same is x
    assert _ulps(out0, F.rms_norm(x, (dim,), w, 1e-6)) <= 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows,inter", [(1, 3072), (64, 3072), (9, 12288), (4, 8)])
def test_silu_mul_matches_torch(dtype, rows, inter):
    torch.manual_seed(rows * 7 + inter)
    gu = (3 * torch.randn(rows, 2 * inter, device=DEV)).to(dtype)
    out = hip_silu_mul(gu)
    gate, up = gu.chunk(2, dim=-1)
    torch_out = F.silu(gate) * up
    assert _ulps(out, torch_out) <= 1
    ref = F.silu(gate.float()) * up.float()
    err = (out.float() - ref).abs()
    assert bool((err <= 1.6e-2 * ref.abs() + 1e-6).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m", [1, 7, 16, 33, 64])
@pytest.mark.parametrize("inter,k", [(3072, 1024), (12288, 4096), (16, 64), (2048, 96)])
def test_linear_swiglu_is_projection_then_gate(dtype, m, inter, k):
    """The fused launch equals hip_silu_mul(hip_linear(x, gate_up)) bit for
    bit (same sums, same rounding steps), and F.silu(gate) * up of the
    float32 product within the 16-bit roundings."""
    torch.manual_seed(m * 31 + inter + k)
    x = torch.randn(m, k, device=DEV).to(dtype)
    w = (0.05 * torch.randn(2 * inter, k, device=DEV)).to(dtype)
    fused = hip_linear_swiglu(x, w)
    assert fused.shape == (m, inter)
    assert torch.equal(fused, hip_silu_mul(hip_linear(x, w)))
    gate, up = _reference(x, w).chunk(2, dim=-1)
    ref = F.silu(gate) * up
    err = (fused.float() - ref).abs()
    assert bool((err <= 2.5e-2 * ref.abs() + 2e-3 * ref.abs().max() + 1e-6).all())
    assert torch.equal(hip_linear_swiglu(x, w), fused)  # reproducible


def test_linear_swiglu_rejects_and_strides():
    w = torch.randn(6144, 1024, device=DEV).to(torch.bfloat16)
    with pytest.raises(ValueError):
        hip_linear_swiglu(torch.randn(65, 1024, device=DEV).to(torch.bfloat16), w)
    with pytest.raises(ValueError):
        hip_linear_swiglu(torch.randn(8, 1024, device=DEV).to(torch.bfloat16), w[:6128])
    torch.manual_seed(9)
    base = torch.randn(24, 1024 + 64, device=DEV).to(torch.bfloat16)
    x = base[:, 64:]
    out = torch.empty(24, 3072 + 32, device=DEV, dtype=torch.bfloat16)[:, :3072]
    y = hip_linear_swiglu(x, w, out=out)
    assert y.data_ptr() == out.data_ptr()
    assert torch.equal(y, hip_silu_mul(hip_linear(x.contiguous(), w)))
