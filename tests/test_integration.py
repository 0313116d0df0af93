"""End-to-end: a small Mamba-2 block and a VMamba path-scan block, HIP kernels against the oracle.

Follows the reference's integration verifier (``benchmarks/verify_cv_integration.py:38-119``):
the same two blocks (in_proj, causal conv1d with SiLU, chunked SSD scan with skip, step bias
and softplus, gated RMSNorm with the gate before the norm, out_proj; and convolutions feeding a
four-path 2D scan), the same loss (the mean square of the block output), and the same checks:
the loss at 5e-5, every parameter gradient at rtol 2e-4 / atol 2e-5, and one SGD step that moves
every parameter.  The reference side here is a float64 copy of each block on the CPU that
calls the float64 oracle; the HIP side is a float32 copy on the GPU calling the public
functions.  NSA block selection, the verifier's third part, is not part of this build.
"""

import copy

import pytest
import torch

import oracle

DEV = "cuda"


class Mamba2Block(torch.nn.Module):
    """The verifier's block (``verify_cv_integration.py:38-78``)."""

    def __init__(self, d_model=24, heads=2, head_dim=6, d_state=5, conv=4, chunk=8):
        super().__init__()
        self.heads, self.head_dim, self.d_state, self.chunk = heads, head_dim, d_state, chunk
        inner = heads * head_dim
        self.inner = inner
        self.in_proj = torch.nn.Linear(d_model, 2 * inner + 2 * d_state + heads)
        self.conv_weight = torch.nn.Parameter(torch.randn(inner + 2 * d_state, 1, conv) * .3)
        self.conv_bias = torch.nn.Parameter(torch.randn(inner + 2 * d_state) * .1)
        self.a_log = torch.nn.Parameter(torch.randn(heads) * .2)
        self.d_skip = torch.nn.Parameter(torch.ones(heads))
        self.dt_bias = torch.nn.Parameter(torch.randn(heads) * .2)
        self.norm_weight = torch.nn.Parameter(torch.ones(inner))
        self.out_proj = torch.nn.Linear(inner, d_model)

    def forward(self, x, reference=False):
        inner, n = self.inner, self.d_state
        zxbcdt = self.in_proj(x)
        z = zxbcdt[..., :inner]
        xbc = zxbcdt[..., inner:2 * inner + 2 * n]
        dt = zxbcdt[..., 2 * inner + 2 * n:]
        weight = self.conv_weight.reshape(inner + 2 * n, -1)
        if reference:
            xbc, _ = oracle.causal_conv1d(xbc.transpose(1, 2), weight, self.conv_bias, "silu")
        else:
            from metal_kernelops.cv import causal_conv1d_fn
            xbc = causal_conv1d_fn(xbc.transpose(1, 2), weight, self.conv_bias, activation="silu")
        xbc = xbc.transpose(1, 2)
        x_ssm = xbc[..., :inner].reshape(x.shape[0], x.shape[1], self.heads, self.head_dim)
        B = xbc[..., inner:inner + n].unsqueeze(2)
        C = xbc[..., inner + n:].unsqueeze(2)
        A = -torch.exp(self.a_log)
        if reference:
            y, _ = oracle.mamba2_chunk_scan_recurrence(x_ssm, dt, A, B, C, D=self.d_skip, dt_bias=self.dt_bias,
                                                       dt_softplus=True)
        else:
            from metal_kernelops.cv import mamba2_chunk_scan
            y, _ = mamba2_chunk_scan(x_ssm, dt, A, B, C, chunk_size=self.chunk, D=self.d_skip,
                                     dt_bias=self.dt_bias, dt_softplus=True)
        y = y.reshape(x.shape[0], x.shape[1], inner)
        if reference:
            y, _ = oracle.rmsnorm_gated(y, self.norm_weight, z=z, norm_before_gate=False)
        else:
            from metal_kernelops.cv import rmsnorm_gated
            y = rmsnorm_gated(y, self.norm_weight, z=z, norm_before_gate=False)
        return self.out_proj(y).square().mean()


class PathBlock(torch.nn.Module):
    """The verifier's VMamba-style block (``verify_cv_integration.py:81-100``)."""

    def __init__(self, channels=6, groups=2, states=4):
        super().__init__()
        self.groups, self.states = groups, states
        self.u = torch.nn.Conv2d(channels, channels, 3, padding=1)
        self.dt = torch.nn.Conv2d(channels, channels, 1)
        self.b = torch.nn.Conv2d(channels, groups * states, 1)
        self.c = torch.nn.Conv2d(channels, groups * states, 1)
        self.a = torch.nn.Parameter(-torch.rand(channels, states))

    def forward(self, x, reference=False):
        u = self.u(x)
        dt = torch.nn.functional.softplus(self.dt(x))
        shape = (x.shape[0], self.groups, self.states, x.shape[2], x.shape[3])
        B, C = self.b(x).reshape(shape), self.c(x).reshape(shape)
        if reference:
            out = oracle.ss2d_scan(u, dt, self.a, B, C, merge="sum")
        else:
            from metal_kernelops.cv import ss2d_scan
            out = ss2d_scan(u, dt, self.a, B, C, merge="sum")
        return out.square().mean()


def _pair(factory):
    torch.manual_seed(17)
    ref = factory().double()
    hip = copy.deepcopy(ref).float().to(DEV)
    return ref, hip


def _check_block(ref, hip, x, loss_tol=5e-5, rtol=2e-4, atol=2e-5):
    """Loss, every parameter gradient, and one SGD step (``verify_cv_integration.py:103-119``)."""
    ref_loss = ref(x, reference=True)
    with torch.backends.cudnn.flags(enabled=False):  # torch's own convolutions, no MIOpen tuning
        hip_loss = hip(x.float().to(DEV))
    ref_loss.backward()
    with torch.backends.cudnn.flags(enabled=False):
        hip_loss.backward()
    torch.testing.assert_close(hip_loss.detach().cpu().double(), ref_loss.detach(), rtol=loss_tol, atol=loss_tol)
    names = []
    for (name, a), (_, b) in zip(ref.named_parameters(), hip.named_parameters()):
        assert b.grad is not None, name
        torch.testing.assert_close(b.grad.cpu().double(), a.grad, rtol=rtol, atol=atol, msg=name)
        names.append(name)
    before = {n: p.detach().clone() for n, p in hip.named_parameters()}
    torch.optim.SGD(ref.parameters(), lr=.03).step()
    torch.optim.SGD(hip.parameters(), lr=.03).step()
    for n, p in hip.named_parameters():
        assert not torch.equal(before[n], p), n
    for (name, a), (_, b) in zip(ref.named_parameters(), hip.named_parameters()):
        torch.testing.assert_close(b.detach().cpu().double(), a.detach(), rtol=rtol, atol=atol, msg=name)
    return names


def test_package_twins_compose_like_the_oracle():
    """The package's pure-torch ``*_reference`` twins give the oracle block's loss on the CPU."""
    from metal_kernelops.cv import causal_conv1d_ref, mamba2_chunk_scan_reference, rmsnorm_gated_reference

    torch.manual_seed(17)
    block = Mamba2Block().double()
    x = torch.randn(2, 19, 24, dtype=torch.float64)
    want = block(x, reference=True)
    inner, n = block.inner, block.d_state
    zxbcdt = block.in_proj(x)
    z, xbc, dt = zxbcdt[..., :inner], zxbcdt[..., inner:2 * inner + 2 * n], zxbcdt[..., 2 * inner + 2 * n:]
    xbc = causal_conv1d_ref(xbc.transpose(1, 2), block.conv_weight.reshape(inner + 2 * n, -1), block.conv_bias,
                            activation="silu").transpose(1, 2)
    x_ssm = xbc[..., :inner].reshape(2, 19, block.heads, block.head_dim)
    y, _ = mamba2_chunk_scan_reference(x_ssm, dt, -torch.exp(block.a_log), xbc[..., inner:inner + n].unsqueeze(2),
                                       xbc[..., inner + n:].unsqueeze(2), chunk_size=8, D=block.d_skip,
                                       dt_bias=block.dt_bias, dt_softplus=True)
    y = rmsnorm_gated_reference(y.reshape(2, 19, inner), block.norm_weight, z=z, norm_before_gate=False)
    got = block.out_proj(y).square().mean()
    assert abs(got.item() - want.item()) < 1e-12


@pytest.mark.gpu
def test_mamba2_block_matches_the_oracle():
    ref, hip = _pair(Mamba2Block)
    x = torch.randn(2, 19, 24, dtype=torch.float64)
    names = _check_block(ref, hip, x)
    assert len(names) == 10


@pytest.mark.gpu
def test_wider_mamba2_block_matches_the_oracle():
    """A wider block: 4 heads of 16, 16 states, 2 x 96 tokens, chunk 32."""
    ref, hip = _pair(lambda: Mamba2Block(d_model=64, heads=4, head_dim=16, d_state=16, conv=4, chunk=32))
    x = torch.randn(2, 96, 64, dtype=torch.float64)
    _check_block(ref, hip, x)


@pytest.mark.gpu
def test_path_block_matches_the_oracle():
    ref, hip = _pair(PathBlock)
    x = torch.randn(2, 6, 9, 11, dtype=torch.float64)
    names = _check_block(ref, hip, x)
    assert len(names) == 9
