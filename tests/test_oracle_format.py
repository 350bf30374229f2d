"""Pins for the INT2 format oracle (oracle/format.py, oracle/store.py,
oracle/rotate.py, oracle/quant_ref.c).

Each check is chosen so a plausible mistake fails it: known-answer bytes
(bit order, LE meta, pad untouched), tie rounding (floor(u + 0.5), not
round-half-even), the 2^-14 scale floor, negative slots, clip index
arithmetic, and the C restatement against the Python one bit-for-bit.
The reference's own checks restated here: constant-vector quantization and
geometry / negative-slot behaviour (tests/test_backend.py:57-73, 152-160),
dequant tolerance 1e-5 (format.py:36).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import format as fmt
from oracle import rotate, store
from oracle.build import build as build_c_oracle


# ---------------------------------------------------------------- known answers
def test_known_answer_codes_and_bytes():
    # min 0, max 3 -> scale 1, zero 0; codes are the values themselves.
    x = torch.tensor([[0.0, 1.0, 2.0, 3.0, 3.0, 2.0, 1.0, 0.0]])
    packed, scale, zero = fmt.quantize(x)
    assert scale.item() == 1.0 and zero.item() == 0.0
    # byte b holds value 4b+k at bits 2k: [0,1,2,3] -> 0b11100100, [3,2,1,0] -> 0b00011011
    assert packed.tolist() == [[0xE4, 0x1B]]
    assert fmt.unpack(packed, 8).tolist() == [[0, 1, 2, 3, 3, 2, 1, 0]]


def test_ties_round_up_not_to_even():
    # (x - 0) / 1 + 0.5 lands exactly on 1.0, 2.0, 3.0: floor gives 1, 2, 3;
    # round-half-even would give 0, 2, 2.  Each step rounds in fp32, so
    # 0.5 - 2^-25 + 0.5 rounds up to 1.0 (q = 1), while 0.5 - 2^-24,
    # 1.5 - 2^-23 and 2.5 - 2^-22 stay just below the next integer.
    e = 2.0 ** -25
    x = torch.tensor([[0.0, 0.5, 1.5, 2.5, 3.0, 0.5 - e, 0.5 - 2 * e, 1.5 - 4 * e, 2.5 - 8 * e]])
    q = fmt.codes(x, *fmt.vector_scales(x))
    assert q.tolist() == [[0, 1, 2, 3, 3, 1, 0, 1, 2]]
    wrong = torch.clamp(torch.round(x), 0, 3).to(torch.int32)
    assert not torch.equal(wrong, q)


def test_f16_little_endian_meta():
    lo, hi = fmt.f16_le(torch.tensor([1.0, -2.0, 2.0 ** -14, 65504.0]))
    assert lo.tolist() == [0x00, 0x00, 0x00, 0xFF] and hi.tolist() == [0x3C, 0xC0, 0x04, 0x7B]
    vals = torch.randn(1000) * 100
    back = fmt.f16_from_le(*fmt.f16_le(vals))
    assert torch.equal(back, vals.to(torch.float16).float())


def test_slot_byte_layout():
    g = torch.Generator().manual_seed(0)
    k, v = torch.randn(3, 2, 256, generator=g), torch.randn(3, 2, 256, generator=g)
    slot = fmt.make_slot_bytes(k, v)
    assert slot.shape == (3, 2, 160)
    assert torch.count_nonzero(slot[..., 8:32]) == 0
    kp, ks, kz = fmt.quantize(k)
    vp, vs, vz = fmt.quantize(v)
    assert torch.equal(slot[..., 32:96], kp) and torch.equal(slot[..., 96:160], vp)
    meta = slot[..., :8].to(torch.int32)
    for j, val in enumerate((ks, kz, vs, vz)):
        bits = val[..., 0].to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
        assert torch.equal(meta[..., 2 * j] | (meta[..., 2 * j + 1] << 8), bits)
    kd, vd = fmt.parse_slot_bytes(slot, 256)
    assert torch.equal(kd, fmt.dequant(kp, ks, kz, 256))
    assert torch.equal(vd, fmt.dequant(vp, vs, vz, 256))


# ---------------------------------------------------------------- closed forms / invariants
@pytest.mark.parametrize("value", [0.0, 1.0, -1.25, 1e-7])
def test_constant_vector_quantization(value):
    x = torch.full((2, 1, 64), value)
    packed, scale, zero = fmt.quantize(x)
    assert torch.isfinite(scale).all() and (scale > 0).all()
    assert torch.equal(scale, torch.full_like(scale, fmt.SCALE_FLOOR))
    out = fmt.dequant(packed, scale, zero, 64)
    torch.testing.assert_close(out, x, atol=1e-5, rtol=1e-3)


def test_scale_floor_is_strict():
    # range exactly 3 * 2^-14 -> (max-min)/3 == 2^-14, not strictly greater -> floor (same value);
    # a slightly larger range passes through the fp16 rounding.
    f = fmt.SCALE_FLOOR
    x = torch.tensor([[0.0, 3 * f, f, 2 * f]])
    s, z = fmt.vector_scales(x)
    assert s.item() == f and z.item() == 0.0
    x = torch.tensor([[0.0, 3 * f * 1.5]])
    s, _ = fmt.vector_scales(x)
    assert s.item() == torch.tensor(1.5 * f).to(torch.float16).float().item()
    x = torch.tensor([[0.0, 3 * f * 0.25]])
    assert fmt.vector_scales(x)[0].item() == f


def test_dequant_error_bound():
    """|x - dequant(quant(x))| <= scale/2 + the fp16 rounding of zero and scale."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, 256, generator=g) * torch.logspace(-3, 2, 4096).unsqueeze(-1)
    p, s, z = fmt.quantize(x)
    err = (fmt.dequant(p, s, z, 256) - x).abs()
    lo, hi = x.amin(-1, keepdim=True), x.amax(-1, keepdim=True)
    exact = (hi - lo) / 3
    slack = (z - lo).abs() + 3 * (s - exact).abs() + 1e-6 * hi.abs().clamp_min(lo.abs())
    assert bool((err <= 0.5 * s + slack).all())


def test_pack_unpack_bijection():
    q = torch.randint(0, 4, (512, 256), dtype=torch.int32, generator=torch.Generator().manual_seed(2))
    p = fmt.pack(q)
    assert torch.equal(fmt.unpack(p, 256), q)
    every = torch.arange(256, dtype=torch.int32)
    codes = torch.stack([(every >> (2 * k)) & 3 for k in range(4)], -1)
    assert torch.equal(fmt.pack(codes.reshape(1, 1024))[0].to(torch.int32), every)


def test_check_d():
    fmt.check_d(256)
    fmt.check_d(32)
    with pytest.raises(ValueError):
        fmt.check_d(258)
    with pytest.raises(ValueError):
        fmt.check_d(260)


# ---------------------------------------------------------------- store / geometry
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.int8])
@pytest.mark.parametrize("hk", [1, 2, 4])
def test_geometry_and_negative_slots(dtype, hk):
    """Restates tests/test_backend.py:57-73 on the oracle store."""
    g = torch.Generator().manual_seed(hk)
    d = 64 if dtype == torch.bfloat16 else 128
    cache = [torch.zeros(8, 4, hk, d, dtype=dtype) for _ in range(2)]
    k, v = torch.randn(3, hk, d, generator=g), torch.randn(3, hk, d, generator=g)
    store.store_ref(k, v, *cache, torch.tensor([-1, 2, -1]))
    expected = [torch.zeros_like(t) for t in cache]
    store.store_ref(k[1:2], v[1:2], *expected, torch.tensor([2]))
    assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(cache, expected))
    before = [t.clone() for t in cache]
    store.store_ref(k, v, *cache, torch.full((3,), -1))
    assert all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(cache, before))


def test_store_matches_logical_slot_and_leaves_pad():
    g = torch.Generator().manual_seed(3)
    kc = torch.full((4, 8, 2, 256), 0x5A, dtype=torch.uint8).view(torch.int8)
    vc = torch.full((4, 8, 2, 256), 0x5A, dtype=torch.uint8).view(torch.int8)
    k, v = torch.randn(5, 2, 256, generator=g), torch.randn(5, 2, 256, generator=g)
    slots = torch.tensor([31, 0, 9, 17, 30])
    store.store_ref(k, v, kc, vc, slots)
    k8, v8 = kc.view(torch.uint8), vc.view(torch.uint8)
    want = fmt.make_slot_bytes(k, v)
    got = store.logical_slots(kc, vc, slots, 2, 256)
    assert torch.equal(got[..., :8], want[..., :8])
    assert torch.equal(got[..., 32:], want[..., 32:])
    page, row = slots // 8, slots % 8
    assert bool((k8[page, row][..., 8:32] == 0x5A).all()) and bool((k8[page, row][..., 96:] == 0x5A).all())
    assert bool((v8[page, row][..., 64:] == 0x5A).all())
    untouched = torch.ones(32, dtype=torch.bool)
    untouched[slots] = False
    assert bool((k8.reshape(32, 2, 256)[untouched] == 0x5A).all())


# ---------------------------------------------------------------- clipping
def test_clip_index_known_answers():
    assert rotate.clip_index(0.96, 256) == 245
    assert rotate.clip_index(0.92, 256) == 235
    assert rotate.clip_index(1.0, 256) == 255
    assert rotate.clip_index(0.5, 8) == 4


def test_clip_small_known_answer_and_identity():
    x = torch.tensor([[1.0, -8.0, 3.0, -2.0, 7.0, 5.0, -6.0, 4.0]])
    # sorted |x| = 1..8, idx 4 -> thr 5
    assert rotate.clip(x, 0.5).tolist() == [[1.0, -5.0, 3.0, -2.0, 5.0, 5.0, -5.0, 4.0]]
    assert rotate.clip(x, 0.0) is x


def test_clip_matches_brute_force_rank():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 256, generator=g)
    for ratio in (0.96, 0.92, 0.5):
        idx = rotate.clip_index(ratio, 256)
        y = rotate.clip(x, ratio)
        for r in range(0, 64, 7):
            a = sorted(abs(float(t)) for t in x[r])
            thr = a[idx]
            assert all(abs(float(t)) <= thr for t in y[r])
            assert sum(abs(float(t)) > thr for t in x[r]) <= 255 - idx


# ---------------------------------------------------------------- C restatement
@pytest.fixture(scope="module")
def c_oracle():
    lib = ctypes.CDLL(str(build_c_oracle()))
    lib.oscar_oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oscar_oracle_f32_to_f16.argtypes = [ctypes.c_float]
    i64, vp = ctypes.c_int64, ctypes.c_void_p
    lib.oscar_oracle_store.restype = ctypes.c_int
    lib.oscar_oracle_store.argtypes = [vp, vp, i64, ctypes.c_int, ctypes.c_int, vp, vp, vp, i64,
                                       i64, i64, i64, i64, i64, i64, ctypes.c_int, ctypes.c_int]
    return lib


def test_c_f32_to_f16_matches_torch(c_oracle):
    g = torch.Generator().manual_seed(5)
    vals = torch.cat([torch.randn(3000, generator=g) * 10 ** torch.randint(-9, 6, (3000,), generator=g),
                      torch.tensor([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25,
                                    3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11])])
    want = vals.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    got = [c_oracle.oscar_oracle_f32_to_f16(float(v)) for v in vals]
    assert got == want.tolist()


@pytest.mark.parametrize("clip", [(0.0, 0.0), (0.96, 0.92)])
def test_c_store_matches_python_store(c_oracle, clip):
    g = torch.Generator().manual_seed(6)
    n, hk, d, bs, pages = 300, 2, 256, 16, 24
    k = (torch.randn(n, hk, d, generator=g) * torch.linspace(0.1, 4, d)).contiguous()
    v = torch.randn(n, hk, d, generator=g).contiguous()
    slots = torch.randperm(pages * bs, generator=g)[:n].to(torch.int64)
    slots[::13] = -1
    kc = [torch.zeros(pages, bs, hk, d, dtype=torch.int8) for _ in range(2)]
    vc = [torch.zeros(pages, bs, hk, d, dtype=torch.int8) for _ in range(2)]
    store.store_ref(rotate.clip(k, clip[0]), rotate.clip(v, clip[1]), kc[0], vc[0], slots)
    ci = [rotate.clip_index(r, d) if r > 0 else -1 for r in clip]
    k8, v8 = kc[1].view(torch.uint8), vc[1].view(torch.uint8)
    rc = c_oracle.oscar_oracle_store(k.data_ptr(), v.data_ptr(), n, hk, d, slots.data_ptr(), k8.data_ptr(),
                                     v8.data_ptr(), bs, *k8.stride()[:3], *v8.stride()[:3], ci[0], ci[1])
    assert rc == 0
    assert torch.equal(kc[0].view(torch.uint8), k8) and torch.equal(vc[0].view(torch.uint8), v8)


# ---------------------------------------------------------------- threshold quantizer derivation
def _round_up_f32(d):
    f = np.float32(d)
    return np.where(f.astype(np.float64) < d, np.nextafter(f, np.float32(np.inf)), f)


def test_threshold_form_equals_floor_form_for_every_fp16_scale():
    """The HIP quantizer replaces q = clamp(floor(fl(fl(t / s) + 0.5)), 0, 3)
    (t = fl(x - zero)) by three comparisons t >= T_j with
        T_1 = ru(s (0.5 - 3 2^-26)), T_2 = ru(s (1.5 - 2^-24)), T_3 = ru(s (2.5 - 2^-23))
    (ru = round up to fp32).  Both forms are monotone in t, so they agree for
    every t exactly when, for each j, t = T_j gives q >= j and the next float
    below T_j gives q < j.  Checked for every normal fp16 scale >= 2^-14."""
    bits = np.arange(0x0400, 0x7C00, dtype=np.uint16)
    s = bits.view(np.float16).astype(np.float32)
    s = s[s >= np.float32(fmt.SCALE_FLOOR)]
    sd = s.astype(np.float64)

    def q_of(t):
        u = (t.astype(np.float32) / s).astype(np.float32)
        return np.clip(np.floor((u + np.float32(0.5)).astype(np.float32)), 0, 3)

    for j, c in ((1, 0.5 - 3 * 2.0 ** -26), (2, 1.5 - 2.0 ** -24), (3, 2.5 - 2.0 ** -23)):
        T = _round_up_f32(sd * c).astype(np.float32)
        below = np.nextafter(T, np.float32(-np.inf))
        assert bool((q_of(T) >= j).all()), f"q >= {j} fails at the threshold"
        assert bool((q_of(below) < j).all()), f"q >= {j} holds below the threshold"
    # A plausible slip — thresholds at s (j - 0.5) exactly — is caught:
    T = _round_up_f32(sd * 0.5).astype(np.float32)
    assert not bool((q_of(np.nextafter(T, np.float32(-np.inf))) < 1).all())
