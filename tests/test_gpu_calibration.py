"""Calibration on the device: the capture hooks and hessians over device
tensors agree with the CPU computation (fp32, relative 1e-4 of the largest
entry), and the quality floor of the composed rotation
(tests/test_numeric.py:309-351 of the reference) holds through the HIP
quantize-write: slot bytes written by the pre-rotated entry are bit-exact
with the oracle's, and their dequantized values give relL2 <= 0.60 after
U @ H @ P_br but >= 1.0 after the plain eigenvector rotation."""
import pytest
import torch

from oracle import format as ofmt
from oracle import store as ostore
from oscar_amd import calib
from oscar_amd import gen_rotations as gr
from oscar_amd.kernels import quant

pytestmark = pytest.mark.gpu

D = 256


def test_device_hessians_match_cpu(device):
    g = torch.Generator().manual_seed(21)
    q = torch.randn(300, 12, D, generator=g)
    k = torch.randn(300, 2, D, generator=g) * 3
    v = torch.randn(300, 2, D, generator=g)
    want = calib.layer_hessians(q, k, v)
    got = calib.layer_hessians(q.to(device), k.to(device), v.to(device))
    for a, b in zip(got, want):
        assert a.device.type == "cuda"
        assert (a.cpu() - b).abs().max() <= 1e-4 * b.abs().max()


def test_quality_floor_through_the_hip_write(device):
    N = 512
    torch.manual_seed(7)
    chan = torch.ones(D)
    chan[:4] = 24.0
    chan[4:12] = 8.0
    chan[12:24] = 2.5
    amp = torch.exp(0.4 * torch.randn(N, 1, 1))
    K = torch.randn(N, 1, D) * chan * amp
    xf = K.reshape(-1, D).float()
    cov = xf.t() @ xf / xf.shape[0]
    evals, evecs = torch.linalg.eigh(cov + 1e-6 * torch.eye(D, dtype=torch.float64))
    order = torch.argsort(evals, descending=True)
    rotations = {"U": evecs[:, order].float().contiguous(),
                 "UHP": gr.compose_rotation(evecs[:, order], evals[order]).float().contiguous()}
    bs, pages = 128, N // 128
    slots = torch.arange(N, dtype=torch.int64)
    rel = {}
    for name, R in rotations.items():
        x = (K @ R).contiguous()
        caches = [torch.zeros(pages, bs, 1, D, dtype=torch.int8, device=device) for _ in range(2)]
        quant.quant_write_prerotated(x.to(device), x.to(device), caches[0], caches[1], slots.to(device), -1, -1)
        torch.cuda.synchronize()
        got = ostore.logical_slots(caches[0].cpu(), caches[1].cpu(), slots, 1, D)
        want = ofmt.make_slot_bytes(x, x)
        assert torch.equal(got, want), name
        rec, _ = ofmt.parse_slot_bytes(got, D)
        rel[name] = ((rec - x).norm() / x.norm()).item()
    assert rel["U"] >= 1.0, rel
    assert rel["UHP"] <= 0.60, rel
