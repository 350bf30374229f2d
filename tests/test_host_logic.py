"""Host-side logic of the drop-in: configuration, rotation checkpoints,
metadata accessors, plugin surgery and memory budgeting.  CPU only; the
library is loaded (no GPU call is made).

Restates the reference's host tests: tests/test_backend.py:108-115 (no device
read of query starts), 135-149 (failed surgery restores class and state),
218-223 (budget), 226-243 (layer verification), 246-252 (strict rotation),
tests/test_numeric.py:172-182, 216-244, 274-296, 369-378, 441-486.
"""
import os
import warnings
from types import SimpleNamespace as NS

import pytest
import torch

from oracle.staging import arena_geometry
from oscar_amd import backend, integration, plugin, rotation
from oscar_amd.backend import OscarAttentionBackendImpl, metadata_batch_lists
from oscar_amd.config import OscarConfig

ENV_KEYS = [k for k in os.environ if k.startswith("OSCAR_ASCEND_")]


@pytest.fixture
def clean_env(monkeypatch):
    for k in ENV_KEYS:
        monkeypatch.delenv(k, raising=False)
    return monkeypatch


# ---------------------------------------------------------------- config
def test_config_defaults(clean_env):
    cfg = OscarConfig.from_env(256)
    assert (cfg.sink_tokens, cfg.recent_tokens, cfg.staging_tokens) == (64, 256, 8192)
    assert cfg.window_enabled and cfg.use_paged
    assert (cfg.k_clip_ratio, cfg.v_clip_ratio) == (0.0, 0.0)
    assert cfg.slot_bytes == 160 and cfg.data_bytes == 64 and cfg.levels == 4


def test_config_env_keys(clean_env):
    clean_env.setenv("OSCAR_ASCEND_K_CLIP_RATIO", "0.96")
    clean_env.setenv("OSCAR_ASCEND_V_CLIP_RATIO", "0.92")
    clean_env.setenv("OSCAR_ASCEND_SINK_TOKENS", "-5")
    clean_env.setenv("OSCAR_ASCEND_RECENT_TOKENS", "0")
    clean_env.setenv("OSCAR_ASCEND_STAGING_TOKENS", "bogus")
    clean_env.setenv("OSCAR_ASCEND_USE_PAGED", "0")
    cfg = OscarConfig.from_env(256)
    assert (cfg.k_clip_ratio, cfg.v_clip_ratio) == (0.96, 0.92)
    assert cfg.sink_tokens == 0 and cfg.staging_tokens == 8192
    assert not cfg.window_enabled and not cfg.use_paged


@pytest.mark.parametrize("value, on", [("1", True), ("0", False), ("false", False), ("off", False),
                                       ("no", False), ("true", False), ("", False), (None, True)])
def test_config_use_paged_as_the_reference_reads_it(clean_env, value, on):
    # config.py:93: a set OSCAR_ASCEND_USE_PAGED is on only for "1"; unset
    # keeps this build's default (on).  VERBOSE stays on unless "0" (:90).
    if value is not None:
        clean_env.setenv("OSCAR_ASCEND_USE_PAGED", value)
        clean_env.setenv("OSCAR_ASCEND_VERBOSE", value)
    cfg = OscarConfig.from_env(256)
    assert cfg.use_paged is on
    assert cfg.verbose is (value != "0")


def test_config_rejections(clean_env):
    clean_env.setenv("OSCAR_ASCEND_K_CLIP_RATIO", "1.5")
    with pytest.raises(ValueError):
        OscarConfig.from_env(256)
    clean_env.setenv("OSCAR_ASCEND_K_CLIP_RATIO", "0.5")
    clean_env.setenv("OSCAR_ASCEND_GROUP_SIZE", "64")
    with pytest.raises(ValueError):
        OscarConfig.from_env(256)


# ---------------------------------------------------------------- rotations
def test_layer_index_from_name():
    assert rotation.layer_index_from_name("model.layers.11.self_attn.attn") == 11
    assert rotation.layer_index_from_name("decoder.block7") == 7
    assert rotation.layer_index_from_name("attn") is None


NOT_V2 = "ignore:OSCAR rotations in .* are not a format-v2"


def test_rotation_loader_warns_on_non_v2_recipes(tmp_path):
    p = tmp_path / "plain.pt"
    torch.save({"layers": {"0": {"rotation": torch.eye(8)}}}, p)
    rotation.load_checkpoint.cache_clear()
    with pytest.warns(UserWarning, match="not a format-v2"):
        rotation.get_layer_rotation(str(p), "model.layers.0.a", 8, "cpu")
    p2 = tmp_path / "v2.pt"
    torch.save({"format_version": 2, "objective": "qqt+sst r_h_pbr", "layers": {"0": {"rotation": torch.eye(8)}}}, p2)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        rotation.get_layer_rotation(str(p2), "model.layers.0.a", 8, "cpu")


@pytest.mark.filterwarnings(NOT_V2)
def test_rotation_checkpoint_formats(tmp_path):
    g = torch.Generator().manual_seed(0)
    R1, R2, R3 = (torch.linalg.qr(torch.randn(64, 64, generator=g)).Q for _ in range(3))
    name = "model.layers.11.self_attn.attn"
    p = tmp_path / "layers.pt"
    torch.save({"layers": {"model.layers.11.self_attn": {"rotation": R1, "rotation_v": R2},
                           "3": {"rotation": R3}}}, p)
    assert torch.equal(rotation.get_layer_rotation(str(p), name, 64, "cpu"), R1)
    assert torch.equal(rotation.get_layer_rotation(str(p), name, 64, "cpu", mode="v"), R2)
    assert torch.equal(rotation.get_layer_rotation(str(p), "model.layers.3.x", 64, "cpu", mode="v"), R3)
    assert torch.equal(rotation.get_layer_rotation(str(p), "model.layers.4.x", 64, "cpu"), torch.eye(64))
    p2 = tmp_path / "flat.pt"
    torch.save({11: R2, "12": {"rotation": R3}}, p2)
    assert torch.equal(rotation.get_layer_rotation(str(p2), name, 64, "cpu"), R2)
    assert torch.equal(rotation.get_layer_rotation(str(p2), "model.layers.12.a", 64, "cpu"), R3)
    p3 = tmp_path / "stacked.pt"
    torch.save(torch.stack([R1, R2, R3]), p3)
    assert torch.equal(rotation.get_layer_rotation(str(p3), "model.layers.2.a", 64, "cpu"), R3)
    assert torch.equal(rotation.get_layer_rotation("", name, 64, "cpu"), torch.eye(64))


@pytest.mark.filterwarnings(NOT_V2)
def test_rotation_strict_mode(tmp_path):
    p = tmp_path / "r.pt"
    torch.save({"layers": {"1": {"rotation": torch.eye(64)}, "2": {"rotation": 2 * torch.eye(64)},
                           "5": {"rotation": torch.eye(32)}}}, p)
    with pytest.raises(ValueError, match="has no rotation for layer"):
        rotation.get_layer_rotation(str(p), "model.layers.0.self_attn.attn", 64, "cpu", strict=True)
    with pytest.raises(ValueError, match="orthogonal"):
        rotation.get_layer_rotation(str(p), "model.layers.2.self_attn.attn", 64, "cpu", strict=True)
    with pytest.raises(ValueError, match="shape"):
        rotation.get_layer_rotation(str(p), "model.layers.5.self_attn.attn", 64, "cpu")


@pytest.mark.filterwarnings(NOT_V2)
def test_rotation_loader_refuses_pickled_objects(tmp_path):
    p = tmp_path / "evil.pt"
    torch.save({"layers": {"1": {"rotation": torch.eye(4), "obj": NS(x=1)}}}, p)
    with pytest.raises(Exception):
        rotation.get_layer_rotation(str(p), "model.layers.1.a", 4, "cpu")


# ---------------------------------------------------------------- metadata
def test_metadata_lists_do_not_read_device_query_starts():
    class NoRead:
        def tolist(self):
            raise AssertionError("unexpected device sync")

    md = NS(query_start_loc=NoRead(), actual_seq_lengths_q=[1, 2], seq_lens=NoRead(), seq_lens_list=[9, 12])
    assert metadata_batch_lists(md) == ([0, 1, 2], [9, 12])


def test_metadata_lists_multi_element_tensors_and_fallbacks():
    m = NS(query_start_loc=torch.tensor([0, 16384, 16389]), query_start_loc_cpu=torch.tensor([0, 16384, 16389]),
           seq_lens=torch.tensor([16384, 5]), seq_lens_cpu=torch.tensor([16384, 5]))
    assert metadata_batch_lists(m) == ([0, 16384, 16389], [16384, 5])
    m2 = NS(query_start_loc=torch.tensor([0, 3]), query_start_loc_cpu=None, seq_lens=torch.tensor([1000]),
            seq_lens_cpu=None)
    assert metadata_batch_lists(m2) == ([0, 3], [1000])
    m3 = NS(query_start_loc=[0, 5], query_start_loc_cpu=None, seq_lens=[8], seq_lens_cpu=None)
    assert metadata_batch_lists(m3) == ([0, 5], [8])
    m4 = NS(query_start_loc=[0, 5], seq_lens=[8], _seq_lens_cpu=torch.tensor([7]))
    assert metadata_batch_lists(m4) == ([0, 5], [7])


# ---------------------------------------------------------------- plugin
def test_failed_surgery_restores_class_and_state():
    class Original:
        pass

    class Broken(Original):
        def _oscar_setup(self):
            self.partial = True
            raise ValueError("unsupported")

    impl = Original()
    impl.keep = 123
    with pytest.raises(ValueError):
        plugin.install_impl(impl, Broken)
    assert type(impl) is Original and vars(impl) == {"keep": 123}


def test_surgery_installs_oscar_over_native_class(clean_env):
    class NativeImpl:
        def __init__(self):
            self.head_size, self.num_heads, self.num_kv_heads = 256, 6, 1
            self.scale = 0.0625

        def forward(self, *a):
            return "native"

    impl = NativeImpl()
    cls = plugin.oscar_class_for(NativeImpl)
    assert plugin.oscar_class_for(NativeImpl) is cls and plugin.oscar_class_for(cls) is cls
    plugin.install_impl(impl, cls)
    assert isinstance(impl, OscarAttentionBackendImpl) and isinstance(impl, NativeImpl)
    assert impl.forward.__func__ is OscarAttentionBackendImpl.forward
    assert impl._oscar.head_dim == 256


def test_surgery_rejects_other_head_sizes(clean_env):
    class NativeImpl:
        head_size, num_heads, num_kv_heads, scale = 128, 8, 1, 0.08

    impl = NativeImpl()
    with pytest.raises(ValueError, match="head_size"):
        plugin.install_impl(impl, plugin.oscar_class_for(NativeImpl))
    assert type(impl) is NativeImpl


def test_hybrid_detection():
    assert plugin._is_hybrid_config(NS(hf_text_config=NS(layer_types=["linear_attention", "attention"])))
    assert not plugin._is_hybrid_config(NS(hf_text_config=NS(layer_types=["attention", "attention"])))
    assert plugin._is_hybrid_config(NS(is_hybrid=True))


def test_mtp_draft_layers_stay_native(capsys):
    plugin._SKIP_REASONS_LOGGED.clear()
    assert plugin._should_oscar(NS(layer_name="model.mtp.layers.0.self_attn.attn"), None) is False
    assert plugin._should_oscar(NS(layer_name="mtp.block.attn"), None) is False
    assert plugin._SKIP_REASONS_LOGGED == {"mtp-draft"}


# ---------------------------------------------------------------- impl host checks
def make_impl(clean_env):
    impl = OscarAttentionBackendImpl.__new__(OscarAttentionBackendImpl)
    impl.head_size, impl.num_kv_heads, impl.num_heads = 256, 1, 6
    impl.scale = 0.0625
    impl.key_cache = impl.value_cache = None
    impl._oscar_setup()
    return impl


def test_cache_geometry_checks(clean_env):
    impl = make_impl(clean_env)
    impl._set_caches([torch.zeros(2, 128, 1, 256, dtype=torch.int8) for _ in range(2)])
    impl._oscar_geo_ok = False
    impl._set_caches([torch.zeros(2, 128, 1, 256, dtype=torch.bfloat16) for _ in range(2)])
    impl._oscar_geo_ok = False
    with pytest.raises(ValueError):
        impl._set_caches([torch.zeros(2, 128, 1, 64, dtype=torch.int8) for _ in range(2)])
    impl._oscar_geo_ok = False
    with pytest.raises(ValueError):
        impl._set_caches([torch.zeros(2, 1, 128, 256, dtype=torch.int8).transpose(1, 2) for _ in range(2)])


def test_forward_without_metadata_zeroes_output(clean_env):
    impl = make_impl(clean_env)
    out = torch.full((3, 6, 256), 5.0)
    caches = [torch.zeros(2, 128, 1, 256, dtype=torch.int8) for _ in range(2)]
    assert torch.count_nonzero(impl.forward(NS(layer_name="l.0"), out, out, out, caches, None, output=out)) == 0


def test_forward_refuses_engine_graph_capture(clean_env, monkeypatch):
    """Launch arguments come from host-side lengths: under capture, forward
    raises unless the caller declared that every replay repeats the step."""
    impl = make_impl(clean_env)
    out = torch.zeros(3, 6, 256)
    caches = [torch.zeros(2, 128, 1, 256, dtype=torch.int8) for _ in range(2)]
    md = NS(attn_state=None)
    monkeypatch.setattr(backend, "_capturing", lambda t: True)
    with pytest.raises(RuntimeError, match="enforce-eager"):
        impl.forward(NS(layer_name="l.0"), out, out, out, caches, md, output=out)
    impl.allow_fixed_step_capture()
    with pytest.raises(NotImplementedError):       # past the check: key = None outside DecodeOnly
        impl.forward(NS(layer_name="l.0"), out, None, None, caches, md, output=out)


def test_forward_without_fresh_kv_needs_the_decode_only_state(clean_env):
    """backend.py:304-309: key = None reads only in the DecodeOnly state, one
    query token per request (checked before any kernel call)."""
    from oscar_amd.backend import OscarAttentionState

    impl = make_impl(clean_env)
    caches = [torch.zeros(2, 128, 1, 256, dtype=torch.int8) for _ in range(2)]
    out = torch.zeros(2, 6, 256)
    md = NS(num_actual_tokens=2, query_start_loc=torch.tensor([0, 2]), seq_lens=torch.tensor([9]),
            seq_lens_list=[9], block_tables=torch.zeros(1, 2, dtype=torch.int32))
    with pytest.raises(NotImplementedError):
        impl.forward(NS(layer_name="l.0"), out, None, None, caches, md, output=out)
    md.attn_state = OscarAttentionState.ChunkedPrefill
    with pytest.raises(NotImplementedError):
        impl.forward(NS(layer_name="l.0"), out, None, None, caches, md, output=out)
    md.attn_state = OscarAttentionState.DecodeOnly
    with pytest.raises(ValueError, match="one query token"):
        impl.forward(NS(layer_name="l.0"), out, None, None, caches, md, output=out)


# ---------------------------------------------------------------- budgeting
def test_budget_accounts_shadow_and_fixed_buffers():
    budget = integration.memory_budget(10000, 100, 25, 1000)
    assert budget == 7200 and budget + (budget // 100) * 25 + 1000 <= 10000
    with pytest.raises(ValueError):
        integration.memory_budget(100, 100, 25, 100)


def test_verify_layers():
    integration.verify_layers(["linear_attention", "full_attention"], [1])
    with pytest.raises(RuntimeError):
        integration.verify_layers(["full_attention"] * 2, [0])
    with pytest.raises(RuntimeError):
        integration.verify_layers(["linear_attention"], [])


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_arena_rows_match_oracle_geometry(bs):
    for sink in (0, 16, 64, 128, 200):
        for recent in (0, 1, 128, 256, 300):
            for staging in (0, 64, 8192):
                assert integration.arena_rows(bs, sink, recent, staging) == arena_geometry(bs, sink, recent,
                                                                                           staging)[3]


def test_plan_capacity_fits_one_mi355x():
    plan = integration.plan_capacity(integration.MI355X_HBM_BYTES - 20 * 10 ** 9, layers=16)
    assert plan["blocks"] * plan["native_per_block"] + plan["fixed"] <= plan["available"]
    assert plan["tokens"] == plan["blocks"] * 128
    # one INT2 token of one layer costs 2 * 256 bytes of int8-geometry slots
    assert plan["native_per_block"] == 2 * 128 * 256 * 16


def test_operand_image_layouts_follow_their_formulas():
    """The fp16 window images the decode reads as MFMA operands, element by element:
    K block m, lane t + 32g, slot u = feature 128g + 16(m // 2) + 4(m % 2) + u // 2 + 8(u % 2)
    of token t; V block (q, b, s), lane m + 32gs, part p, slot u = feature 64q + 4(m // 2) + 2b + m % 2
    of token 16s + 8gs + (0, 2, 1, 3, 4, 6, 5, 7)[u].  Each image's second part holds
    fp16(x - fp16(x)) (K: a second image in the same order; V: the 8 halves after the lane's
    high part), so that the two parts sum to x within 2^-22 |x| + 2^-25 (half the spacing of
    fp16 subnormals, where the low part of a small x lies)."""
    from oscar_amd.kernels import staging as kstaging

    g = torch.Generator().manual_seed(3)
    sk = torch.randn(2, 64, 1, 256, generator=g)
    sv = torch.randn(2, 64, 1, 256, generator=g)
    kimg, vimg = kstaging.stage_images(sk, sv)
    order = [0, 2, 1, 3, 4, 6, 5, 7]
    for r, tile in ((0, 0), (1, 1)):
        K, KL = kimg[r, tile, 0].view(2, 16, 64, 8)
        V = vimg[r, tile, 0].view(4, 2, 2, 64, 2, 8)
        for lane in range(64):
            t, gg = lane % 32, lane // 32
            for m in range(16):
                for u in range(8):
                    f = 128 * gg + 16 * (m // 2) + 4 * (m % 2) + u // 2 + 8 * (u % 2)
                    x = sk[r, 32 * tile + t, 0, f]
                    assert K[m, lane, u] == x.half()
                    assert KL[m, lane, u] == (x - x.half().float()).half()
                    assert abs(K[m, lane, u].double() + KL[m, lane, u].double() - x.double()) <= 2.0 ** -22 * abs(x) + 2.0 ** -25
            mm, gs = lane % 32, lane // 32
            for q in range(4):
                for b in range(2):
                    for s in range(2):
                        for u in range(8):
                            f = 64 * q + 4 * (mm // 2) + 2 * b + mm % 2
                            tok = 16 * s + 8 * gs + order[u]
                            x = sv[r, 32 * tile + tok, 0, f]
                            hi, lo = V[q, b, s, lane, 0, u], V[q, b, s, lane, 1, u]
                            assert hi == x.half() and lo == (x - x.half().float()).half()
                            assert abs(hi.double() + lo.double() - x.double()) <= 2.0 ** -22 * abs(x) + 2.0 ** -25


def test_request_layout_is_built_once_per_step():
    """The layers of a step share one validated layout; new lengths build a new one."""
    from oscar_amd.kernels import decode as kdecode

    a = kdecode.request_layout([0, 4, 5], [100, 7])
    assert kdecode.request_layout((0, 4, 5), (100, 7)) is a
    assert a.lengths == [4, 1] and a.max_q == 4 and a.max_hist == 96
    assert list(a.qstart) == [0, 4, 5] and list(a.seq_t) == [100, 7]
    b = kdecode.request_layout([0, 4, 5], [101, 7])
    assert b is not a and b.max_hist == 97
    with pytest.raises(ValueError):
        kdecode.request_layout([0, 4, 5], [3, 7])         # history would be negative


class _RecordingLib:
    """The real library for its host-only size queries; the MTP forward entry
    replaced by a recorder (no kernel is called without a GPU)."""

    def __init__(self, real):
        self._real = real
        self.calls = []

    def __getattr__(self, name):
        return getattr(self._real, name)

    def oscar_mtp_forward(self, layer, st, q, qs, k, v, ks, out, os_, bf16, stream):
        self.calls.append(dict(layer=layer, step=st, q=q, qs=qs, k=k, v=v, ks=ks, out=out, os=os_, bf16=bf16))
        return 0


def _short_step_setup(clean_env, monkeypatch):
    from oscar_amd.kernels import _lib, step as kstep

    real = _lib.load()
    fake = _RecordingLib(real)
    monkeypatch.setattr(_lib, "_lib", fake)
    monkeypatch.setattr(_lib, "stream_handle", lambda dev: 1234)
    monkeypatch.setattr(kstep, "_LAST_STEP", [None])
    impls, layers = [], []
    for i in range(2):
        impl = make_impl(clean_env)
        layer = NS(layer_name=f"model.layers.{i}.self_attn.attn")
        rk, rv = torch.eye(256), torch.eye(256)
        layer._oscar_rots = (rk, rv)
        layer._oscar_rot_ops = (rk, rv, None, None)
        layer._oscar_rvT = rv.t().contiguous()
        impls.append(impl)
        layers.append(layer)
    caches = [[torch.zeros(8, 128, 1, 256, dtype=torch.int8) for _ in range(2)] for _ in range(2)]
    return fake, impls, layers, caches


def _short_md(seqs, qlens):
    qsl = [0]
    for n in qlens:
        qsl.append(qsl[-1] + n)
    N = qsl[-1]
    return NS(num_actual_tokens=N, slot_mapping=torch.arange(N, dtype=torch.int64),
              query_start_loc_cpu=torch.tensor(qsl, dtype=torch.int32), seq_lens_list=list(seqs),
              block_tables=torch.zeros(len(seqs), 8, dtype=torch.int32), attn_state=None)


def test_short_step_packs_layer_and_step_halves_once(clean_env, monkeypatch):
    """Every layer of a short step makes one oscar_mtp_forward call; the
    layers share the step half, and each layer's half is packed once and
    reused by the next step."""
    fake, impls, layers, caches = _short_step_setup(clean_env, monkeypatch)
    md = _short_md([300, 41], [4, 1])
    q = torch.zeros(7, 6 * 256, dtype=torch.bfloat16)       # 2 padding rows
    kv = torch.zeros(7, 3 * 256, dtype=torch.bfloat16)      # k | v | pad columns of a fused projection
    k, v = kv[:, :256], kv[:, 256:512]
    outs = [torch.full((7, 6 * 256), 3.0, dtype=torch.bfloat16) for _ in range(2)]
    for impl, layer, c, out in zip(impls, layers, caches, outs):
        impl.forward(layer, q, k, v, c, md, output=out)
    assert len(fake.calls) == 2
    a, b = fake.calls
    assert a["step"] == b["step"] and a["layer"] != b["layer"]
    assert a["qs"] == 6 * 256 and a["ks"] == 3 * 256 and a["v"] == v.data_ptr() and a["bf16"] == 1
    assert a["out"] == outs[0].data_ptr() and a["os"] == 6 * 256
    for out in outs:
        assert (out[5:] == 0).all() and (out[:5] == 3.0).all()   # padding rows cleared, the rest left to the kernel
    # The next step: new lengths build a new step half; the layer halves stay.
    md2 = _short_md([301, 42], [1, 1])
    for impl, layer, c, out in zip(impls, layers, caches, outs):
        impl.forward(layer, q, k, v, c, md2, output=out)
    c, d = fake.calls[2:]
    assert c["step"] == d["step"] != a["step"]
    assert c["layer"] == a["layer"] and d["layer"] == b["layer"]
    # A rebound cache rebuilds that layer's half.
    caches[0] = [t.clone() for t in caches[0]]
    impls[0].forward(layers[0], q, k, v, caches[0], md2, output=outs[0])
    assert fake.calls[-1]["layer"] != a["layer"] and fake.calls[-1]["step"] == c["step"]


def test_short_step_routing_and_capture(clean_env, monkeypatch):
    """A request longer than 16 tokens leaves the short route; under a
    declared fixed-step capture every call builds its own step half (its
    scratch then belongs to the graph)."""
    fake, impls, layers, caches = _short_step_setup(clean_env, monkeypatch)
    impl, layer, c = impls[0], layers[0], caches[0]
    q = torch.zeros(17, 6 * 256, dtype=torch.bfloat16)
    k = torch.zeros(17, 256, dtype=torch.bfloat16)
    out = torch.zeros(17, 6 * 256, dtype=torch.bfloat16)
    impl._set_caches(c)
    assert impl._short_step(layer, q, k, k, c, _short_md([300], [17]), out, False) is False
    assert fake.calls == []
    from oscar_amd.kernels import step as kstep

    built = []
    init = kstep.MtpStep.__init__
    monkeypatch.setattr(kstep.MtpStep, "__init__", lambda self, *a: (built.append(1), init(self, *a))[1])
    monkeypatch.setattr(kstep, "_LAST_STEP", [None])
    md = _short_md([300], [4])
    assert impl._short_step(layer, q, k, k, c, md, out, True) is True
    assert impl._short_step(layer, q, k, k, c, md, out, True) is True
    assert len(built) == 2 and kstep._LAST_STEP[0] is None and len(fake.calls) == 2
    assert impl._short_step(layer, q, k, k, c, md, out, False) is True
    assert impl._short_step(layer, q, k, k, c, md, out, False) is True
    assert len(built) == 3 and fake.calls[2]["step"] == fake.calls[3]["step"]


def test_bench_profile_figures_need_unchanged_sources(tmp_path, monkeypatch):
    """bench.py reports a committed rocprofv3 figure only while every source it
    was measured on hashes as recorded; a changed source turns it into null."""
    import hashlib

    import bench

    src = tmp_path / "oscar_amd" / "csrc"
    src.mkdir(parents=True)
    (src / "k.hip").write_text("kernel v1\n")
    (tmp_path / "profiles").mkdir()
    digest = hashlib.sha256(b"kernel v1\n").hexdigest()
    (tmp_path / "profiles" / "t.txt").write_text(
        f"header line: not a figure\nfigure traffic C2: 1234\nsource_sha256 k.hip: {digest}\n")
    monkeypatch.setattr(bench, "ROOT", tmp_path)
    assert bench.profile_figures("t.txt") == {"traffic C2": 1234.0}
    (src / "k.hip").write_text("kernel v2\n")
    assert bench.profile_figures("t.txt") == {}
    assert bench.profile_figures("missing.txt") == {}


@pytest.mark.parametrize("q_lens,hist", [
    ([4], [24579]),                                          # one request, one step per split
    ([1] * 8, [32768] * 8),                                  # 8 x 256 steps: 4 steps per split, 512 splits
    ([4] * 32, [2048 + 448 * i for i in range(32)]),         # mixed lengths
    ([1] * 3, [300000, 5, 0]),                               # a long request, a tiny one and an empty one
])
def test_decode_split_plan_invariants(q_lens, hist):
    """Restated split plan (paged_decode.hip plan_splits): every split takes
    at most 64 steps (one page-register lane each), no item gets more splits
    than steps, the history splits stay within one round of resident
    workgroups when 64 steps per split allow it, and the partial slots fit the
    workspace bound."""
    nsplit, pbase = integration.decode_split_plan(q_lens, hist, max(hist))
    steps = [-(-h // integration.DECODE_STEP) for h in hist]
    for n, s in zip(nsplit, steps):
        assert n <= s
        if s:
            assert n >= 1 and -(-s // n) <= integration.DECODE_MAX_STEPS_PER_SPLIT
    if sum(-(-s // integration.DECODE_MAX_STEPS_PER_SPLIT) for s in steps) <= integration.DECODE_RESIDENT_SPLITS:
        assert sum(nsplit) <= integration.DECODE_RESIDENT_SPLITS
    assert pbase[-1] + nsplit[-1] + 1 <= integration.decode_partial_slots(len(hist), max(hist))


def test_decode_split_plan_leaves_a_one_tile_last_step_uncounted():
    """8 DecodeOnly reads of 32769 positions: 257 steps, the last holding one
    token.  Counting it would need 5 steps per split (52 splits per item);
    leaving it out gives 64 splits of 4 steps (split 0 also takes the short
    step), 512 workgroups in all.  A last step of 33 tokens is counted."""
    nsplit, _ = integration.decode_split_plan([1] * 8, [32769] * 8, 32769, fresh=0)
    assert nsplit == [64] * 8
    nsplit, _ = integration.decode_split_plan([1] * 8, [32768 + 33] * 8, 32768 + 33, fresh=0)
    assert nsplit == [52] * 8
