"""GPTQ (nibblegemm_amd.gptq): the column-loop kernel against the CPU oracle,
the oracle against exact arithmetic, and the properties the reference's own
tests hold the algorithm to (tests/test_gptq.py in the reference: the output
format, beating round-to-nearest on output error while losing on weight
error, the identity-Hessian limit, dead channels, singular Hessians, the
Hessian accumulator).

The product runs its column loop on the GPU only, so everything that calls
``gptq_quantize`` is marked ``gpu``; the accumulator, the argument checks, the
model-walking helpers and the oracle run on the CPU.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
import nibblegemm_amd as ng
from nibblegemm_amd import gptq
from nibblegemm_amd.gptq import HessianAccumulator, _inverse_cholesky, gptq_quantize

dev = "cuda"


def make_layer(K, N, seed=0, device="cpu"):
    """A weight and a *correlated* activation distribution (with white
    activations the Hessian is near-diagonal and GPTQ reduces to RTN, which
    would prove nothing) -- the reference test's construction
    (tests/test_gptq.py:17-31)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    mix = torch.randn(K, K, generator=g) * 0.1 + torch.eye(K)
    X = torch.randn(2048, K, generator=g) @ mix
    X[:, : max(1, K // 32)] *= 6.0
    W = torch.randn(K, N, generator=g) * 0.02
    W[torch.rand(K, N, generator=g) < 0.002] *= 10
    H = 2.0 * (X.t() @ X) / X.shape[0]
    return W.to(device), X.to(device), H.to(device)


def output_mse(W_ref, X, qw):
    return (X @ ng.dequantize(qw).float() - X @ W_ref).pow(2).mean().item()


def weight_mse(W_ref, qw):
    return (ng.dequantize(qw).float() - W_ref).pow(2).mean().item()


# ---------------------------------------------------------------------------
# The oracle's column loop, pinned
# ---------------------------------------------------------------------------
def exact_group(w_rows, U):
    """The recurrence in exact rational arithmetic (scale = amax / 7 exactly,
    q = nearest integer, ties to even), for inputs chosen away from rounding
    ties so float32 must make the same decisions."""
    G = len(U)
    out = []
    for row in w_rows:
        w = [Fraction(x) for x in row]
        scale = max(abs(x) for x in w) / 7
        qs, errs = [], []
        for i in range(G):
            q = max(-8, min(7, round(w[i] / scale)))
            err = (w[i] - q * scale) / Fraction(U[i][i])
            for j in range(i + 1, G):
                w[j] -= err * Fraction(U[i][j])
            qs.append(q + 8)
            errs.append(err)
        out.append((qs, errs, scale))
    return out


def test_oracle_group_loop_matches_exact_arithmetic():
    """Three channels whose compensation changes the rounding: transposing U,
    dropping the 1/U[i][i] or flipping the update's sign each change q."""
    U = np.array([[0.5, 1.5, -0.75], [0.0, 0.4, 2.0], [0.0, 0.0, 1.0]], dtype=np.float32)
    W = np.array([[-0.51, 0.54, -0.58], [0.66, -0.87, 0.65], [-0.67, -0.25, -0.37]],
                 dtype=np.float32)
    qu, err, sc = oracle.gptq_group(W, U)
    for n, (q_ex, e_ex, s_ex) in enumerate(exact_group(W.tolist(), U.tolist())):
        assert qu[n].tolist() == q_ex, (n, qu[n], q_ex)
        # float32 cancellation in w - q * scale: agreement to 1e-5 absolute
        # (a formula mistake moves err by a sizeable fraction of the ~0.1 scale)
        assert np.allclose(err[n], [float(e) for e in e_ex], rtol=0, atol=1e-5)
        assert sc[n] == pytest.approx(float(s_ex), rel=1e-6)
    # the mutations the example is built to catch all change some nibble
    for bad in (U.T.copy(), np.diag(np.diag(U)), U * np.where(np.eye(3), 1, -1)):
        assert not np.array_equal(oracle.gptq_group(W, bad.astype(np.float32))[0], qu)


def test_oracle_group_loop_structure():
    """Rows are independent (a row permutation permutes the outputs), only
    U's upper triangle is read, and a diagonal U means no compensation: each
    channel is rounded on its own with the group's scale."""
    rng = np.random.default_rng(0)
    N, G = 37, 16
    W = (rng.standard_normal((N, G)) * 0.02).astype(np.float32)
    U = np.triu(rng.standard_normal((G, G)) * 0.1).astype(np.float32) + np.eye(G, dtype=np.float32)
    qu, err, sc = oracle.gptq_group(W, U)
    perm = rng.permutation(N)
    q2, e2, s2 = oracle.gptq_group(W[perm], U)
    assert np.array_equal(q2, qu[perm]) and np.array_equal(e2, err[perm])
    assert np.array_equal(s2, sc[perm])
    q3, e3, _ = oracle.gptq_group(W, U + np.tril(rng.standard_normal((G, G)), -1).astype(np.float32))
    assert np.array_equal(q3, qu) and np.array_equal(e3, err)
    qd, _, sd = oracle.gptq_group(W, np.eye(G, dtype=np.float32))
    inv = (np.float32(1) / sd)[:, None]
    assert np.array_equal(qd, (np.clip(np.rint(W * inv), -8, 7) + 8).astype(np.uint8))


# ---------------------------------------------------------------------------
# Host-side pieces (CPU)
# ---------------------------------------------------------------------------
def test_hessian_accumulator_matches_direct_computation():
    K = 32
    X = torch.randn(500, K)
    acc = HessianAccumulator(K, device="cpu")
    for start in range(0, 500, 64):
        acc.add(X[start:start + 64])
    torch.testing.assert_close(acc.H, 2.0 * (X.t() @ X) / X.shape[0], rtol=1e-4, atol=1e-4)


def test_hessian_accumulator_flattens_leading_dims():
    """Hooks see [batch, seq, features]; both leading dimensions are rows."""
    acc = HessianAccumulator(16, device="cpu")
    acc.add(torch.randn(4, 8, 16))
    assert acc.n == 32


def test_hessian_accumulator_ignores_empty_batches():
    acc = HessianAccumulator(16, device="cpu")
    acc.add(torch.randn(0, 16))
    assert acc.n == 0 and torch.equal(acc.H, torch.zeros(16, 16))


def test_inverse_cholesky_is_upper_triangular():
    """Upper triangular with a positive diagonal, and U^T U is the damped
    inverse (float64, so the reconstruction is checked tightly)."""
    _, _, H = make_layer(128, 32)
    U = _inverse_cholesky(H.double(), damp=0.01, retries=3)
    assert torch.equal(U, torch.triu(U)) and bool((torch.diag(U) > 0).all())
    lam = 0.01 * torch.diag(H.double()).mean()
    torch.testing.assert_close(U.t() @ U, torch.linalg.inv(H.double() + lam * torch.eye(128)))


def test_rejects_shape_mismatch():
    W, _, H = make_layer(256, 64)
    with pytest.raises(ValueError):
        gptq_quantize(W, H[:128, :128], group_size=128)
    with pytest.raises(ValueError):
        gptq_quantize(W, H, group_size=100)


class _Block(nn.Module):
    def __init__(self, d, ff):
        super().__init__()
        self.up = nn.Linear(d, ff, bias=False)
        self.down = nn.Linear(ff, d, bias=True)
        self.odd = nn.Linear(d, 6)  # N % 4 != 0: not supported by the kernels

    def forward(self, x):
        return x + self.down(torch.relu(self.up(x))) + 0 * self.odd(x).sum(-1, keepdim=True)


class _Toy(nn.Module):
    def __init__(self, d=256, ff=512, n=2):
        super().__init__()
        self.model = nn.Module()
        self.model.layers = nn.ModuleList([_Block(d, ff) for _ in range(n)])

    def forward(self, x):
        for blk in self.model.layers:
            x = blk(x)
        return x


def test_find_decoder_blocks_and_supported_linear():
    toy = _Toy()
    assert gptq.find_decoder_blocks(toy) is toy.model.layers
    assert gptq.find_decoder_blocks(nn.Linear(4, 4)) is None
    assert gptq.supported_linear(nn.Linear(256, 512), 128)
    assert not gptq.supported_linear(nn.Linear(256, 6), 128)
    assert not gptq.supported_linear(nn.Linear(200, 512), 128)


# ---------------------------------------------------------------------------
# The kernel (GPU)
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("G", [64, 128])
@pytest.mark.parametrize("N", [1, 63, 64, 65, 300])
def test_group_kernel_is_the_oracle_bit_for_bit(G, N):
    rng = np.random.default_rng(G + N)
    K = 2 * G
    Wt = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    Wt[rng.random((N, K)) < 0.01] *= 10
    A = rng.standard_normal((K, K)).astype(np.float32) * 0.1
    U = np.triu(A) + np.eye(K, dtype=np.float32) * 2.0
    # the second group of the row block: exercises the row and factor strides
    i1 = G
    q_ref, e_ref, s_ref = oracle.gptq_group(Wt[:, i1:i1 + G], U[i1:i1 + G, i1:i1 + G])
    ext = ng.extension()
    Wd = torch.from_numpy(Wt).to(dev)
    Ud = torch.from_numpy(U).to(dev)
    Q = torch.zeros((N, K), dtype=torch.uint8, device=dev)
    E = torch.empty((N, G), dtype=torch.float32, device=dev)
    S = torch.empty(N, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    rc = ext.gptq_group(Wd.data_ptr() + 4 * i1, K, N, G, Ud.data_ptr() + 4 * (i1 * K + i1), K,
                        Q.data_ptr() + i1, K, E.data_ptr(), S.data_ptr(), stream)
    assert rc == 0, ext.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(Q[:, i1:].cpu().numpy(), q_ref)
    assert bool((Q[:, :i1] == 0).all())  # nothing written outside the group's columns
    assert np.array_equal(E.cpu().numpy(), e_ref)
    assert np.array_equal(S.cpu().numpy(), s_ref)
    assert torch.equal(Wd.cpu(), torch.from_numpy(Wt))  # the input is only read


def test_group_kernel_rejections():
    ext = ng.extension()
    P = 1 << 20
    assert ext.gptq_group(P, 128, 10, 96, P, 128, P, 128, P, P, None) == 1
    assert "group size" in ext.last_error()
    assert ext.gptq_group(P, 64, 10, 128, P, 128, P, 128, P, P, None) == 1
    assert "leading" in ext.last_error()
    assert ext.gptq_group(0, 128, 0, 128, 0, 128, 0, 128, 0, 0, None) == 0  # no rows


# ---------------------------------------------------------------------------
# gptq_quantize (GPU)
# ---------------------------------------------------------------------------
@pytest.mark.gpu
@pytest.mark.parametrize("K,N,G", [(128, 64, 128), (64, 300, 64)])
def test_single_group_is_the_oracle_bit_for_bit(K, N, G):
    """One group: no inter-group product, so the whole quantisation is the
    column loop on the factor -- bit for bit the oracle's."""
    W, _, H = make_layer(K, N, seed=K + N)
    qw = gptq_quantize(W.to(dev), H.to(dev), group_size=G)
    U = _inverse_cholesky(H.to(dev).float().clone(), 0.01, 5).cpu().numpy()
    qu, sc = oracle.gptq_quantize(W.numpy(), U, G)
    assert np.array_equal(ng.unpack_nibbles(qw.qweight.numpy(), K), qu)
    assert np.array_equal(qw.scales.numpy(), sc.astype(np.float16))


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,G", [(512, 128, 128), (512, 96, 64)])
def test_multi_group_tracks_the_oracle(K, N, G):
    """Later groups see the earlier groups' errors through a float32 product
    (hipBLASLt here, BLAS in the oracle).  The two summation orders flip rare
    near-tie roundings, and a flip changes that row's later compensation, so
    the check is a small mismatch fraction and an equally good result."""
    W, X, H = make_layer(K, N, seed=3)
    qw = gptq_quantize(W.to(dev), H.to(dev), group_size=G)
    U = _inverse_cholesky(H.to(dev).float().clone(), 0.01, 5).cpu().numpy()
    qu, sc = oracle.gptq_quantize(W.numpy(), U, G)
    got = ng.unpack_nibbles(qw.qweight.numpy(), K)
    assert (got != qu).mean() < 1e-2
    assert np.allclose(qw.scales.float().numpy(), sc, rtol=1e-2)
    ref_qw = ng.QuantizedWeight(torch.from_numpy(ng.pack_nibbles(qu)),
                                torch.from_numpy(sc.astype(np.float16)), G, K, N)
    assert output_mse(W, X, qw) == pytest.approx(output_mse(W, X, ref_qw), rel=0.02)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N,G", [(256, 64, 128), (512, 128, 64), (384, 32, 128)])
def test_output_format_matches_quantize(K, N, G):
    W, _, H = make_layer(K, N)
    qw = gptq_quantize(W, H, group_size=G)
    ref = ng.quantize(W, group_size=G)
    assert qw.qweight.shape == ref.qweight.shape == (K // 8, N)
    assert qw.scales.shape == ref.scales.shape == (K // G, N)
    assert qw.qweight.dtype == torch.int32 and qw.scales.dtype == torch.float16
    assert (qw.K, qw.N, qw.group_size) == (K, N, G)


@pytest.mark.gpu
def test_packed_values_are_four_bit():
    W, _, H = make_layer(256, 64)
    qw = gptq_quantize(W, H, group_size=128)
    nib = ng.unpack_nibbles(qw.qweight.numpy(), qw.K)
    assert nib.min() >= 0 and nib.max() <= 15


@pytest.mark.gpu
def test_scales_are_positive_and_finite():
    W, _, H = make_layer(256, 64)
    s = gptq_quantize(W, H, group_size=128).scales.float()
    assert bool(torch.isfinite(s).all()) and bool((s > 0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", [(256, 64), (512, 128)])
def test_beats_rtn_on_output_error(K, N):
    """The objective GPTQ minimises: error at the layer's output."""
    W, X, H = make_layer(K, N)
    rtn = ng.quantize(W, group_size=128)
    assert output_mse(W, X, gptq_quantize(W, H, group_size=128)) < output_mse(W, X, rtn)


@pytest.mark.gpu
@pytest.mark.parametrize("K,N", [(256, 64), (512, 128)])
def test_is_worse_on_weight_error(K, N):
    """Compensation moves weights further from their originals on purpose: a
    later channel's error cancels an earlier one's at the output."""
    W, _, H = make_layer(K, N)
    rtn = ng.quantize(W, group_size=128)
    assert weight_mse(W, gptq_quantize(W, H, group_size=128)) > weight_mse(W, rtn)


@pytest.mark.gpu
def test_identity_hessian_is_rounding_with_the_group_scale():
    """A diagonal Hessian couples no channels: the factor is diagonal and
    GPTQ rounds every weight on its own with scale amax * fp32(1/7)."""
    K, N = 256, 64
    W, _, _ = make_layer(K, N)
    q = gptq_quantize(W, torch.eye(K) * 2.0, group_size=128)
    groups = W.reshape(K // 128, 128, N)
    scale = (groups.abs().amax(dim=1) * np.float32(1.0 / 7.0)).clamp(min=1e-8)
    expect = (torch.round(groups * (1.0 / scale).unsqueeze(1)).clamp(-8, 7) + 8).reshape(K, N)
    assert np.array_equal(ng.unpack_nibbles(q.qweight.numpy(), K), expect.to(torch.uint8).numpy())


@pytest.mark.gpu
def test_identity_hessian_stays_close_to_rtn():
    """The reference's looser form of the identity-Hessian limit."""
    K, N = 256, 64
    W, _, _ = make_layer(K, N)
    g = ng.dequantize(gptq_quantize(W, torch.eye(K) * 2.0, group_size=128)).float()
    r = ng.dequantize(ng.quantize(W, group_size=128)).float()
    assert float((g - r).abs().max() / r.abs().max()) < 0.5


@pytest.mark.gpu
def test_dead_channels_are_handled():
    """A channel no calibration token activated makes H singular; it is zeroed."""
    K, N = 256, 64
    W, _, H = make_layer(K, N)
    H[10, :] = 0
    H[:, 10] = 0
    q = gptq_quantize(W, H, group_size=128)
    assert bool(torch.isfinite(q.scales.float()).all())
    assert ng.dequantize(q)[10].abs().max().item() == 0.0


@pytest.mark.gpu
def test_singular_hessian_escalates_damping():
    """A rank-4 Hessian still yields finite weights (damping grows until the
    factorisation succeeds)."""
    base = torch.randn(128, 4, generator=torch.Generator().manual_seed(3))
    q = gptq_quantize(make_layer(128, 32)[0], base @ base.t(), group_size=128)
    assert bool(torch.isfinite(ng.dequantize(q).float()).all())


@pytest.mark.gpu
def test_kernel_runs_on_gptq_weights():
    K, N = 512, 128
    W, _, H = make_layer(K, N)
    qw = gptq_quantize(W, H, group_size=128).to(dev)
    X = torch.randn(1, K, dtype=torch.float16, device=dev)
    ref = ng.reference_matmul(X.cpu(), qw.to("cpu")).to(dev)
    got = ng.gemv(X, qw, version=4)
    assert float((got.float() - ref.float()).abs().max() / ref.float().pow(2).mean().sqrt()) < 1e-2


@pytest.mark.gpu
def test_quantize_model_gptq_replaces_supported_linears():
    torch.manual_seed(0)
    toy = _Toy().to(dev).half()
    calib = [torch.randn(4, 16, 256, device=dev).half() for _ in range(3)]
    x = torch.randn(2, 8, 256, device=dev).half()
    with torch.no_grad():
        ref = toy(x).float()
    logs = []
    n, skipped = gptq.quantize_model_gptq(toy, calib, group_size=128, log=logs.append)
    assert n == 4 and len(skipped) == 2 and all("odd" in s for s in skipped)
    assert len(logs) == 2
    for blk in toy.model.layers:
        assert isinstance(blk.up, ng.QuantLinear) and isinstance(blk.down, ng.QuantLinear)
        assert isinstance(blk.odd, nn.Linear)
    with torch.no_grad():
        y = toy(x).float()
    assert float((y - ref).abs().max() / ref.abs().max()) < 0.1
