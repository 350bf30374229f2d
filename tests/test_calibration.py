"""Rotation calibration (oscar_amd.calib, oscar_amd.gen_rotations), CPU.

Pinned by what the mathematics fixes rather than by retyping the formulas:
the Sylvester Hadamard recursion and orthogonality, bit reversal as an
involution with known small cases, P_br moving the i-th largest eigenvector
to column bitrev(i), U^T Sigma U diagonal for the U recovered from R, the
hessians' invariants (scale invariance of the score weights, isotropic
queries reducing Sigma_S to the plain second moment, identical kv heads
reducing to one head), the count-weighted merge, the format-v2 round trip
through the product loader, and the reference's quality floor
(tests/test_numeric.py:309-351): per-vector INT2 over outlier channels is
noise-level after the plain eigenvector rotation and within relL2 0.60 after
U @ H @ P_br.  The whole tool runs once against a fake vLLM engine.
"""
import json
import sys
from types import ModuleType
import warnings
from types import SimpleNamespace as NS

import pytest
import torch

from oracle import format as ofmt
from oscar_amd import calib, plugin, rotation
from oscar_amd import gen_rotations as gr


# ---------------------------------------------------------------- composition
def test_hadamard_sylvester_and_orthogonal():
    assert torch.equal(gr.hadamard(1), torch.ones(1, 1, dtype=torch.float64))
    s = 2 ** -0.5
    assert torch.allclose(gr.hadamard(2), torch.tensor([[s, s], [s, -s]], dtype=torch.float64))
    for n in (4, 16, 256):
        h = gr.hadamard(n)
        assert torch.allclose(h @ h.t(), torch.eye(n, dtype=torch.float64), atol=1e-12)
        assert torch.allclose(h.abs(), torch.full((n, n), n ** -0.5, dtype=torch.float64))
        m = gr.hadamard(n // 2) * s
        assert torch.allclose(h, torch.cat([torch.cat([m, m], 1), torch.cat([m, -m], 1)], 0))
    for bad in (0, 3, 12):
        with pytest.raises(ValueError):
            gr.hadamard(bad)


def test_bit_reversal_known_cases_and_involution():
    assert gr.bit_reversal_perm(1).tolist() == [0]
    assert gr.bit_reversal_perm(2).tolist() == [0, 1]
    assert gr.bit_reversal_perm(8).tolist() == [0, 4, 2, 6, 1, 5, 3, 7]
    p = gr.bit_reversal_perm(256)
    assert torch.equal(p[p], torch.arange(256))
    assert p[1].item() == 128 and p[255].item() == 255
    with pytest.raises(ValueError):
        gr.bit_reversal_perm(6)


def test_br_permutation_places_largest_directions_at_bit_reversed_columns():
    evals = torch.tensor([1.0, 5.0, 3.0, 2.0], dtype=torch.float64)
    P = gr.br_permutation(evals)
    M = torch.arange(16, dtype=torch.float64).reshape(4, 4)
    # descending order 1, 2, 3, 0 placed at columns bitrev(0..3) = 0, 2, 1, 3
    assert torch.equal((M @ P)[:, [0, 2, 1, 3]], M[:, [1, 2, 3, 0]])
    assert torch.equal(P.sum(0), torch.ones(4, dtype=torch.float64))
    assert torch.equal(P.sum(1), torch.ones(4, dtype=torch.float64))


def random_spd(D, seed, outliers=4):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(4 * D, D, generator=g, dtype=torch.float64)
    x[:, :outliers] *= 10
    return x.t() @ x / x.shape[0]


def test_rotation_from_stats_diagonalises_the_hessian():
    D = 64
    cov = random_spd(D, 1)
    R, evals = gr.rotation_from_stats({"cov_sum": (cov * 7).float(), "count": 7}, D)
    R64 = R.double()
    assert (R64 @ R64.t() - torch.eye(D, dtype=torch.float64)).abs().max() < 1e-5
    # undo P_br and H: U = R P_br^T H^T has the eigenvectors as columns
    U = R64 @ gr.br_permutation(evals.double()).t() @ gr.hadamard(D).t()
    inner = U.t() @ cov.float().double() @ U
    off = inner - torch.diag(torch.diagonal(inner))
    assert off.abs().max() < 1e-4 * cov.abs().max()
    assert torch.allclose(torch.diagonal(inner), evals.double() - 1e-6, rtol=1e-4, atol=1e-5)
    assert torch.all(evals[1:] >= evals[:-1])


def test_quality_floor_outlier_channels():
    """tests/test_numeric.py:309-351 on the same synthetic recipe."""
    D, N = 256, 512
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
    U_old = evecs[:, order].float().contiguous()
    R_new = gr.compose_rotation(evecs[:, order], evals[order], gr.hadamard(D)).float().contiguous()
    assert (R_new @ R_new.t() - torch.eye(D)).abs().max().item() < 1e-4

    def rel(x_rot):
        packed, scale, zero = ofmt.quantize(x_rot.float())
        rec = ofmt.dequant(packed, scale, zero, D)
        return ((rec - x_rot).norm() / x_rot.norm()).item()

    r_old, r_new = rel(K @ U_old), rel(K @ R_new)
    assert r_old >= 1.0, r_old
    assert r_new <= 0.60, r_new


# ---------------------------------------------------------------- hessians
def captures(n, hq, hk, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, hq, D, generator=g), torch.randn(n, hk, D, generator=g),
            torch.randn(n, hk, D, generator=g))


def test_sigma_q_is_the_mean_query_second_moment():
    q, k, v = captures(9, 6, 1, 16, 1)
    sq, _ = calib.layer_hessians(q, k, v)
    rows = q.reshape(-1, 16).double()
    want = sum(torch.outer(r, r) for r in rows) / rows.shape[0]
    assert torch.allclose(sq.double(), want, rtol=1e-5, atol=1e-6)


def test_score_weights_are_scale_invariant_and_isotropic_queries_reduce_sigma_s():
    n, D = 8, 16
    q, k, v = captures(n, 2, 1, D, 2)
    sq, ss = calib.layer_hessians(q, k, v)
    sq2, ss2 = calib.layer_hessians(3 * q, 0.5 * k, v)
    assert torch.allclose(sq2, 9 * sq, rtol=1e-5) and torch.allclose(ss2, ss, rtol=1e-4, atol=1e-6)
    # queries whose second moment is a multiple of I and keys of equal norm: w = 1
    qi = torch.eye(D)[:, None, :].expand(D, 2, D)
    kk = torch.nn.functional.normalize(torch.randn(D, 1, D, generator=torch.Generator().manual_seed(3)), dim=-1)
    vv = torch.randn(D, 1, D, generator=torch.Generator().manual_seed(4))
    _, ss_iso = calib.layer_hessians(qi.contiguous(), kk, vv)
    plain = vv[:, 0].double().t() @ vv[:, 0].double() / D
    assert torch.allclose(ss_iso.double(), plain, rtol=1e-4, atol=1e-6)
    # zero keys: all weights vanish
    _, ss0 = calib.layer_hessians(q, torch.zeros_like(k), v)
    assert torch.count_nonzero(ss0) == 0


def test_identical_kv_heads_match_one_head():
    q1, k1, v1 = captures(7, 3, 1, 16, 5)
    q2 = torch.cat([q1, q1], 1)
    k2, v2 = torch.cat([k1, k1], 1), torch.cat([v1, v1], 1)
    a = calib.layer_hessians(q1, k1, v1)
    b = calib.layer_hessians(q2, k2, v2)
    assert all(torch.allclose(x, y, rtol=1e-5, atol=1e-7) for x, y in zip(a, b))
    # groups are contiguous: heads 0..2 belong to kv head 0
    q3 = torch.cat([q1, 2 * q1], 1)
    sq3, _ = calib.layer_hessians(q3, k2, v2)
    assert torch.allclose(sq3, 2.5 * a[0], rtol=1e-5, atol=1e-6)


def test_merge_weights_by_token_count():
    D = 4
    a = {"l": {"q": {"cov": torch.eye(D), "count": 3}, "v": {"cov": 2 * torch.eye(D), "count": 3}}}
    b = {"l": {"q": {"cov": 5 * torch.eye(D), "count": 1}, "v": {"cov": torch.zeros(D, D), "count": 1}}}
    m = gr.merge_rank_stats([a, b], D)
    assert m["l"]["q"]["count"] == 4 and torch.allclose(m["l"]["q"]["cov_sum"] / 4, 2 * torch.eye(D))
    assert torch.allclose(m["l"]["v"]["cov_sum"] / 4, 1.5 * torch.eye(D))


def test_checkpoint_round_trip_through_the_loader(tmp_path, capsys):
    D = 256
    stats = {}
    for lid, seed in ((3, 11), (7, 12)):
        stats[f"model.layers.{lid}.self_attn.attn"] = {
            "q": {"cov_sum": random_spd(D, seed).float() * 5, "count": 5},
            "v": {"cov_sum": random_spd(D, seed + 50).float() * 5, "count": 5}}
    stats["lm_head.attn"] = stats["model.layers.3.self_attn.attn"]
    ckpt = gr.build_checkpoint(stats, D)
    assert sorted(ckpt["layers"]) == ["3", "7"] and ckpt["format_version"] == 2
    path = tmp_path / "rot.pt"
    torch.save(ckpt, path)
    rotation.load_checkpoint.cache_clear()
    with warnings.catch_warnings():
        warnings.simplefilter("error")          # a format-v2 checkpoint loads without the recipe warning
        for lid in (3, 7):
            name = f"model.layers.{lid}.self_attn.attn"
            rk = rotation.get_layer_rotation(str(path), name, D, "cpu", mode="k", strict=True)
            rv = rotation.get_layer_rotation(str(path), name, D, "cpu", mode="v", strict=True)
            assert torch.equal(rk, ckpt["layers"][str(lid)]["rotation"])
            assert torch.equal(rv, ckpt["layers"][str(lid)]["rotation_v"])
            assert not torch.equal(rk, rv)
    with pytest.raises(ValueError, match="has no rotation for layer"):
        rotation.get_layer_rotation(str(path), "model.layers.0.self_attn.attn", D, "cpu", strict=True)
    rotation.load_checkpoint.cache_clear()
    with pytest.raises(ValueError):
        gr.build_checkpoint({"lm_head.attn": stats["lm_head.attn"]}, D)


# ---------------------------------------------------------------- capture hooks
class FakeAttention(torch.nn.Module):
    def __init__(self, layer_name, hq=4, hk=2, D=8):
        super().__init__()
        self.layer_name, self.num_heads, self.num_kv_heads, self.head_size = layer_name, hq, hk, D

    def forward(self, q, k, v):
        return q


@pytest.fixture
def fresh_captures(monkeypatch):
    monkeypatch.setattr(calib, "_captures", {})
    monkeypatch.setattr(calib, "_REGISTERED", set())
    monkeypatch.setattr(calib, "_TOKEN_CAP", 10)


def test_hooks_capture_head_views_up_to_the_cap(fresh_captures):
    full = FakeAttention("model.layers.0.self_attn.attn")
    skipped = [FakeAttention("model.layers.1.linear_attn.attn"), FakeAttention("model.mtp.layers.0.self_attn.attn"),
               FakeAttention("model.layers.2.mlp")]
    for m in [full, full] + skipped:
        calib.register_attention_hook(m)
    g = torch.Generator().manual_seed(0)
    batches = [torch.randn(n, 4 * 8, generator=g) for n in (6, 7)]
    for x in batches:
        full(x, x[:, :16], x[:, 16:])
        for m in skipped:
            m(x, x[:, :16], x[:, 16:])
    assert list(calib._captures) == ["model.layers.0.self_attn.attn"]
    got = calib._captures["model.layers.0.self_attn.attn"]
    assert [t.shape for t in got["q"]] == [(6, 4, 8), (4, 4, 8)]
    assert [t.shape for t in got["k"]] == [(6, 2, 8), (4, 2, 8)]
    assert torch.equal(got["v"][1], batches[1][:4, 16:].reshape(4, 2, 8))
    out = calib.finalize_cov()
    st = out["model.layers.0.self_attn.attn"]
    assert st["q"]["count"] == 10 and st["q"]["cov"].shape == (8, 8)
    q = torch.cat([batches[0], batches[1][:4]]).reshape(10, 4, 8)
    kv = torch.cat([batches[0], batches[1][:4]])
    want = calib.layer_hessians(q, kv[:, :16].reshape(10, 2, 8), kv[:, 16:].reshape(10, 2, 8))
    assert torch.allclose(st["q"]["cov"], want[0]) and torch.allclose(st["v"]["cov"], want[1])
    calib.reset_captures()
    assert calib.finalize_cov() == {}


def test_plugin_calibration_mode_hooks_without_swapping(monkeypatch, fresh_captures):
    class Attention(FakeAttention):
        def __init__(self, layer_name):
            super().__init__(layer_name)
            self.impl = NS()

    module = ModuleType("vllm.attention.layer")
    module.Attention = Attention
    monkeypatch.setitem(sys.modules, "vllm.attention.layer", module)
    monkeypatch.setattr(plugin, "_PATCHED", False)
    monkeypatch.setenv("OSCAR_ASCEND_CALIB", "1")
    monkeypatch.setenv("OSCAR_ASCEND_ENABLE", "0")
    plugin.load_plugin()
    layer = Attention("model.layers.5.self_attn.attn")
    assert type(layer.impl) is NS
    x = torch.randn(3, 32)
    layer(x, x[:, :16], x[:, 16:])
    assert "model.layers.5.self_attn.attn" in calib._captures


# ---------------------------------------------------------------- the tool
def test_gen_rotations_end_to_end_on_a_fake_engine(monkeypatch, tmp_path, fresh_captures, capsys):
    """main(): calibration env, engine arguments, reset -> generate -> finalize
    through apply_model, merge over two fake workers, checkpoint on disk."""
    D = 256
    monkeypatch.setattr(calib, "_TOKEN_CAP", 512)
    layers = [FakeAttention(f"model.layers.{i}.self_attn.attn", hq=6, hk=1, D=D) for i in (3, 7)]
    for m in layers:
        calib.register_attention_hook(m)
    seen = {}

    class LLM:
        def __init__(self, **kwargs):
            seen["kwargs"] = kwargs
            seen["env"] = {k: __import__("os").environ.get(k) for k in ("OSCAR_ASCEND_CALIB", "OSCAR_ASCEND_ENABLE")}
            self.llm_engine = NS(apply_model=lambda fn: [fn(None), fn(None)])

        def generate(self, prompt, params):
            seen["prompt"] = prompt
            g = torch.Generator().manual_seed(1)
            for m in layers:
                x = torch.randn(100, 6 * D, generator=g)
                kv = torch.randn(100, 2 * D, generator=g)
                m(x, kv[:, :D], kv[:, D:])

    fake = ModuleType("vllm")
    fake.LLM, fake.SamplingParams = LLM, lambda **kw: kw
    monkeypatch.setitem(sys.modules, "vllm", fake)
    monkeypatch.setenv("OSCAR_ASCEND_ENABLE", "1")
    monkeypatch.setenv("OSCAR_ASCEND_GEN_LLM_ARGS", json.dumps({"max_num_seqs": 4}))
    # main() sets these itself; registering them here restores them afterwards
    monkeypatch.setenv("OSCAR_ASCEND_CALIB", "0")
    monkeypatch.setenv("VLLM_WORKER_MULTIPROC_METHOD", "spawn")
    monkeypatch.setenv("VLLM_ALLOW_INSECURE_SERIALIZATION", "1")
    out = tmp_path / "sub" / "rot.pt"
    assert gr.main(["--model", "/models/x", "--save", str(out)]) == 0
    assert seen["env"] == {"OSCAR_ASCEND_CALIB": "1", "OSCAR_ASCEND_ENABLE": None}
    assert seen["kwargs"]["tensor_parallel_size"] == 1 and seen["kwargs"]["max_num_seqs"] == 4
    assert seen["kwargs"]["max_model_len"] == 144 and len(seen["prompt"]) == 120
    ckpt = torch.load(out, weights_only=True)
    assert sorted(ckpt["layers"]) == ["3", "7"]
    r = ckpt["layers"]["3"]["rotation"]
    assert (r @ r.t() - torch.eye(D)).abs().max() < 1e-4
    # the two fake workers saw the same captures: the merge is their mean
    st = calib.finalize_cov()["model.layers.3.self_attn.attn"]
    want, _ = gr.rotation_from_stats({"cov_sum": st["q"]["cov"] * 100, "count": 100}, D)
    assert torch.allclose(r, want, atol=1e-5)
