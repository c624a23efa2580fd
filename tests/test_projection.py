"""The projection GEMMs' split weight gradient (prospective_rqf_amd/projection.py).

``weight_grad`` must equal the single GEMM it replaces, ``g @ x^H``
(rqf_models/ops/selective_scan.py:145; the autograd of ``W @ h``), for every
split count, with and without a remainder of columns; the autograd wrappers
must give what torch's own autograd of the plain products gives
(``_SplitProjection``, rqf_models/backbones/rqf/selective.py:78-97).  These run
on the CPU: the helpers are device-agnostic torch code around library GEMMs.
"""

import numpy as np
import pytest
import torch

from prospective_rqf_amd.projection import (
    WGRAD_MIN_COLUMNS,
    project,
    split_projection,
    weight_grad,
)


def _rand(shape, complex_, gen):
    if complex_:
        return torch.complex(torch.randn(*shape, generator=gen), torch.randn(*shape, generator=gen))
    return torch.randn(*shape, generator=gen)


@pytest.mark.parametrize("complex_", [True, False])
@pytest.mark.parametrize("m,k,n,splits", [
    (5, 3, 4096, 128),       # 4 splits of 1024, no remainder
    (5, 3, 4100, 128),       # 4 splits + 4 remainder columns
    (7, 4, 1000, 128),       # below the split threshold: one GEMM
    (8, 6, 300000, 128),     # 128 splits + remainder
    (3, 2, 9000, 3),         # explicit split count
    (2, 2, 2048, 2),
])
def test_weight_grad_equals_the_single_gemm(complex_, m, k, n, splits):
    gen = torch.Generator().manual_seed(m * 100 + n)
    g, x = _rand((m, n), complex_, gen), _rand((k, n), complex_, gen)
    want = g.numpy().astype(np.complex128 if complex_ else np.float64)
    xs = x.numpy().astype(want.dtype)
    want = want @ (xs.conj().T if complex_ else xs.T)
    got = weight_grad(g, x, splits=splits).numpy()
    assert got.shape == (m, k)
    err = np.abs(got - want).max() / np.abs(want).max()
    assert err < 2e-6, err


def test_weight_grad_rejects_mismatched_shapes():
    with pytest.raises(ValueError):
        weight_grad(torch.zeros(3, 10), torch.zeros(2, 11))
    with pytest.raises(ValueError):
        weight_grad(torch.zeros(3, 10, 1), torch.zeros(2, 10))


def test_split_path_is_deterministic_and_uses_non_contiguous_inputs():
    gen = torch.Generator().manual_seed(1)
    g = _rand((4, 2 * WGRAD_MIN_COLUMNS * 3 + 7), True, gen)
    x = _rand((3, g.shape[1]), True, gen)
    a = weight_grad(g, x)
    b = weight_grad(g.clone(), x.clone())
    assert torch.equal(a, b)
    # A transposed (non-contiguous) operand gives the same result.
    c = weight_grad(g.T.contiguous().T, x)
    assert torch.equal(a, c)


@pytest.mark.parametrize("complex_", [True, False])
def test_project_autograd_matches_plain_matmul(complex_):
    gen = torch.Generator().manual_seed(3)
    dt = torch.complex128 if complex_ else torch.float64
    W = _rand((6, 5), complex_, gen).to(dt).requires_grad_(True)
    h = _rand((5, 3 * WGRAD_MIN_COLUMNS + 11), complex_, gen).to(dt).requires_grad_(True)
    g = _rand((6, h.shape[1]), complex_, gen).to(dt)
    y = project(W, h)
    y.backward(g)
    W2, h2 = W.detach().clone().requires_grad_(True), h.detach().clone().requires_grad_(True)
    (W2 @ h2).backward(g)
    assert torch.allclose(y, W2 @ h2)
    assert torch.allclose(W.grad, W2.grad, rtol=1e-12, atol=1e-9)
    assert torch.allclose(h.grad, h2.grad, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("sizes", [(3, 2, 4), (0, 2, 4), (3, 0, 4), (3, 2, 0)])
def test_split_projection_matches_reference_semantics(sizes):
    gen = torch.Generator().manual_seed(5)
    n = 2 * WGRAD_MIN_COLUMNS + 3
    v = torch.randn(6, n, generator=gen, dtype=torch.float64).requires_grad_(True)
    rows = sum(sizes)
    Ws = torch.randn(rows, 6, generator=gen, dtype=torch.float64).requires_grad_(True)
    outs = split_projection(v, Ws, sizes)
    assert [o.shape[0] for o in outs] == list(sizes)
    # Only some heads receive a cotangent (the reference fills the rest with zeros).
    loss = sum((o * torch.linspace(-1, 1, o.numel(), dtype=o.dtype).reshape(o.shape)).sum()
               for i, o in enumerate(outs) if i != 1 and o.numel())
    if not isinstance(loss, torch.Tensor):
        pytest.skip("no head with a cotangent")
    loss.backward()
    v2, W2 = v.detach().clone().requires_grad_(True), Ws.detach().clone().requires_grad_(True)
    outs2 = (W2 @ v2).split(sizes)
    loss2 = sum((o * torch.linspace(-1, 1, o.numel(), dtype=o.dtype).reshape(o.shape)).sum()
                for i, o in enumerate(outs2) if i != 1 and o.numel())
    loss2.backward()
    assert torch.allclose(v.grad, v2.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(Ws.grad, W2.grad, rtol=1e-12, atol=1e-9)


def test_stacked_reads_consecutive_blocks_in_place():
    from prospective_rqf_amd.projection import stacked

    buf = torch.arange(2 * 7 * 5, dtype=torch.float32).reshape(7, 2, 5)  # (rows, B, T)
    a, b, c = buf[:3], buf[3:4], buf[4:]
    s = stacked([a, b, c])
    assert s.data_ptr() == buf.data_ptr() and s.shape == (7, 10)
    assert torch.equal(s, buf.reshape(7, 10))
    # Not consecutive: a copy with the same values.
    s2 = stacked([c, a])
    assert s2.data_ptr() != buf.data_ptr()
    assert torch.equal(s2, torch.cat([c.reshape(3, 10), a.reshape(3, 10)]))
    assert stacked([None, buf[:0]]) is None


def test_stacked_does_not_join_separate_allocations():
    from prospective_rqf_amd.projection import stacked

    # Two tensors that happen to be adjacent in memory but have separate storages.
    big = torch.zeros(10, 4)
    a = big[:3].clone()
    b = torch.ones(2, 4)
    s = stacked([a, b])
    assert s.shape == (5, 4) and torch.equal(s, torch.cat([a, b]))


def _kernel_emulation(packed, b_cplx, b_real, out_cplx_rows, out_real_rows):
    """What rqf_proj_gemm computes, in fp64 on the CPU: B rows from the interleaved
    complex rows then the real rows, C = A B, C rows scattered to complex then real."""
    rows = []
    if b_cplx is not None:
        rows.append(torch.view_as_real(b_cplx.to(torch.complex128)).permute(0, 2, 1)
                    .reshape(-1, b_cplx.shape[1]))
    if b_real is not None:
        rows.append(b_real.double())
    b = torch.cat(rows, 0)
    a = packed.double()[:b.shape[0]].T  # (m_pad, K)
    c = a @ b
    zc = None
    if out_cplx_rows:
        pairs = c[:2 * out_cplx_rows].reshape(out_cplx_rows, 2, -1)
        zc = torch.complex(pairs[:, 0], pairs[:, 1])
    return zc, c[2 * out_cplx_rows:2 * out_cplx_rows + out_real_rows]


def test_packed_weights_give_the_reference_products():
    from prospective_rqf_amd.projection import pack_dx, pack_forward
    from prospective_rqf_amd.readout import pack_feature_grad, pack_hidden

    gen = torch.Generator().manual_seed(11)
    F, D, ml, N = 5, 3, 7, 13
    W = _rand((F, D), True, gen)
    Ws = torch.randn(ml, 2 * D, generator=gen)
    x = _rand((D, N), True, gen)
    x64, W64, Ws64 = x.to(torch.complex128), W.to(torch.complex128), Ws.double()
    v = torch.cat((x64.real, x64.imag), 0)
    z, lg = _kernel_emulation(pack_forward(W, Ws), x, None, F, ml)
    assert torch.allclose(z, W64 @ x64, atol=1e-9) and torch.allclose(lg, Ws64 @ v, atol=1e-9)
    dz = _rand((F, N), True, gen)
    g = torch.randn(ml, N, generator=gen)
    dx, _ = _kernel_emulation(pack_dx(W, Ws), dz, g, D, 0)
    dv = Ws64.T @ g.double()
    want = W64.mH @ dz.to(torch.complex128) + torch.complex(dv[:D], dv[D:])
    assert torch.allclose(dx, want, atol=1e-9)
    # Readout: hidden = W1 [Re f; Im f]; the feature gradient W1^T dh as complex rows.
    H = 4
    w1 = torch.randn(H, 2 * F, generator=gen)
    f = _rand((F, N), True, gen)
    _, hid = _kernel_emulation(pack_hidden(w1), f, None, 0, H)
    f64 = f.to(torch.complex128)
    assert torch.allclose(hid, w1.double() @ torch.cat((f64.real, f64.imag), 0), atol=1e-9)
    dh = torch.randn(H, N, generator=gen)
    df, _ = _kernel_emulation(pack_feature_grad(w1), None, dh, F, 0)
    dfv = w1.double().T @ dh.double()
    assert torch.allclose(df, torch.complex(dfv[:F], dfv[F:]), atol=1e-9)
