"""Launches follow the current stream of the tensors' device, and a training step run on a
non-default stream gives the bits of the default stream's (the reference's
sparse_pooling/tests/test_device_runtime.py:99-113 test_nondefault_stream, whose deterministic
reduction asserts bitwise equality; every HIP reduction here has a fixed order)."""
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a ROCm GPU")]

from granulelayer_amd import FusedAdamW, SparsePoolingLayer  # noqa: E402
from granulelayer_amd.backend import HipBackend  # noqa: E402

DEV = "cuda"


def _step(lay, opt, x, dy):
    """forward, backward into main_grad, FusedAdamW; returns (y, dX, dW, db, W', b')."""
    x = x.clone().requires_grad_(True)
    y = lay(x)
    y.backward(dy)
    grads = (lay.weight.main_grad.clone(), lay.bias.main_grad.clone())
    opt.step()
    return (y.detach(), x.grad, *grads, lay.weight.detach().clone(), lay.bias.detach().clone())


@pytest.mark.parametrize("pooling", ["sum", "max", {"type": "logmeanexp", "temperature": 0.5}],
                         ids=["sum", "max", "lme"])
def test_nondefault_stream_gives_the_default_streams_bits(pooling, monkeypatch):
    lay = SparsePoolingLayer(1024, 200_000, 64, shared_neurons=None, pooling=pooling, dtype=torch.float32,
                             device=DEV, seed=4, bias_std=0.2)
    lay.enable_main_grad()
    w0, b0 = lay.weight.detach().clone(), lay.bias.detach().clone()
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(256, 1024, generator=gen).to(DEV)
    dy = torch.randn(256, 64, generator=gen).to(DEV)

    opt = FusedAdamW([lay.weight, lay.bias], lr=1e-3, moments="fp32")
    ref = _step(lay, opt, x, dy)
    torch.cuda.synchronize()

    # the same step from the same state, on another stream
    with torch.no_grad():
        lay.weight.copy_(w0)
        lay.bias.copy_(b0)
    lay.zero_main_grad()
    opt = FusedAdamW([lay.weight, lay.bias], lr=1e-3, moments="fp32")
    be = HipBackend.get()
    streams = []
    call = be.lib.call

    def spy(name, *args):
        if name in ("gl_fwd", "gl_bwd", "gl_adam"):
            streams.append((name, args[-1].value))
        return call(name, *args)

    monkeypatch.setattr(be.lib, "call", spy)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        got = _step(lay, opt, x, dy)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    names = [n for n, _ in streams]
    assert "gl_fwd" in names and "gl_bwd" in names and "gl_adam" in names, names
    assert all(v == s.cuda_stream for _, v in streams), streams
    for name, a, b in zip(("y", "dX", "dW", "db", "W", "b"), ref, got):
        assert torch.equal(a, b), f"{name} differs between the default and a non-default stream"
