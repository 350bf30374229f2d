"""GPU parity of kernel 1 (quantize-write) against the CPU oracle.

* Pre-rotated entry: cache bytes bit-exact with the oracle store given the
  same rotated fp32 input (whole caches compared, so pad bytes and bytes of
  skipped slots must be untouched).
* Fused entry (MFMA rotation): the rotation is computed in a different order
  than the oracle's fp32 CPU matmul, so codes may differ only where a rotated
  value sits within rounding distance of a bin edge.  Tolerances, stated:
  >= 99.9 % of code bytes identical, every dequantized value within one
  quantization step (max of the two scales) of the oracle's, meta scale within
  2 fp16 ulps.
"""
import pytest
import torch

from oracle import format as ofmt
from oracle import rotate as orot
from oracle import store as ostore
from oscar_amd import synthetic
from oscar_amd.kernels import quant

pytestmark = pytest.mark.gpu

D = 256


def make_caches(pages, bs, hk, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    width = D if dtype == torch.int8 else D
    raw = torch.randint(0, 256, (2, pages, bs, hk, width * (1 if dtype == torch.int8 else 2)),
                        generator=g, dtype=torch.uint8)
    return [raw[i].view(dtype).clone() for i in range(2)]


def zero_sign_free(c8: torch.Tensor) -> torch.Tensor:
    """K-cache bytes with each slot's zero meta (bytes 2:4 K zero, 6:8 V zero)
    written as +0 where it is fp16 -0.  A vector whose clip threshold is 0 has
    zero = +-0: torch's clamp and amin leave the sign of that zero to the
    memory layout (two layouts of the same values give different signs), so
    the tests compare it as a value."""
    out = c8.clone()
    for off in (2, 6):
        neg = (out[..., off] == 0) & (out[..., off + 1] == 0x80)
        out[..., off + 1][neg] = 0
    return out


def oracle_store(k_rot, v_rot, caches, slots, ck, cv):
    out = [c.clone() for c in caches]
    N, hk, _ = k_rot.shape
    kr = orot.clip(k_rot, ck)
    vr = orot.clip(v_rot, cv)
    ostore.store_ref(kr, vr, out[0], out[1], slots)
    return out


@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.bfloat16])
@pytest.mark.parametrize("hk", [1, 2])
@pytest.mark.parametrize("ratios", [(0.96, 0.92), (0.0, 0.0), (0.5, 0.75), (1.0, 0.004)])
def test_prerotated_bit_exact(device, cache_dtype, hk, ratios):
    torch.manual_seed(0)
    N, bs, pages = 300, 128, 6
    k, v = synthetic.kv(N, hk, D, seed=11)
    Rk, Rv = synthetic.rotations(D, seed=5)
    k_rot = k.float() @ Rk
    v_rot = v.float() @ Rv
    perm = torch.randperm(pages * bs, generator=torch.Generator().manual_seed(3))[:N]
    slots = perm.to(torch.int64)
    slots[::7] = -1
    caches = make_caches(pages, bs, hk, cache_dtype, seed=9)
    expect = oracle_store(k_rot, v_rot, caches, slots, *ratios)
    dev = [c.to(device) for c in caches]
    quant.quant_write_prerotated(k_rot.to(device), v_rot.to(device), dev[0], dev[1], slots.to(device),
                                 quant.clip_index(ratios[0], D), quant.clip_index(ratios[1], D))
    torch.cuda.synchronize()
    for got, want in zip(dev, expect):
        diff = (got.cpu().view(torch.uint8) != want.view(torch.uint8)).sum().item()
        assert diff == 0, f"{diff} bytes differ"


def test_prerotated_edge_vectors(device):
    """Constant vectors, ties at the clip threshold, exact bin edges, tiny ranges."""
    hk, bs = 1, 16
    rows = []
    rows.append(torch.zeros(D))
    rows.append(torch.full((D,), 1.0))
    rows.append(torch.full((D,), -1.25))
    rows.append(torch.full((D,), 1e-7))
    x = torch.linspace(-3, 3, D)
    rows.append(x)
    rows.append(torch.round(x * 4) / 4)          # many ties
    rows.append(torch.tensor([0.5, -0.5] * (D // 2)))
    ramp = torch.arange(D, dtype=torch.float32) / 85.0   # values on exact bin edges
    rows.append(ramp)
    rows.append(1000.0 + torch.arange(D) * 1e-4)        # tiny range at large magnitude
    rows.append(torch.where(torch.arange(D) % 2 == 0, 1.0, -1.0) * 65000.0)
    k_rot = torch.stack(rows).unsqueeze(1).float()
    v_rot = k_rot.flip(0).clone()
    N = k_rot.shape[0]
    slots = torch.arange(N, dtype=torch.int64)
    for ratios in [(0.96, 0.92), (0.0, 0.0), (0.5, 0.5)]:
        caches = [torch.zeros(2, bs, hk, D, dtype=torch.int8) for _ in range(2)]
        expect = oracle_store(k_rot, v_rot, caches, slots, *ratios)
        dev = [c.to(device) for c in caches]
        quant.quant_write_prerotated(k_rot.to(device), v_rot.to(device), dev[0], dev[1], slots.to(device),
                                     quant.clip_index(ratios[0], D), quant.clip_index(ratios[1], D))
        torch.cuda.synchronize()
        for got, want in zip(dev, expect):
            assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8)), ratios


def test_prerotated_large_random_write(device):
    """65,536-token write with random slots and ~1/16 skipped (C5 write shape)."""
    N, hk, bs = 65536, 1, 128
    pages = N // bs + 8
    g = torch.Generator().manual_seed(21)
    k_rot = torch.randn(N, hk, D, generator=g) * 1.7
    v_rot = torch.randn(N, hk, D, generator=g)
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int64)
    slots[torch.rand(N, generator=g) < 1 / 16] = -1
    caches = [torch.zeros(pages, bs, hk, D, dtype=torch.int8) for _ in range(2)]
    expect = oracle_store(k_rot, v_rot, caches, slots, 0.96, 0.92)
    dev = [c.to(device) for c in caches]
    quant.quant_write_prerotated(k_rot.to(device), v_rot.to(device), dev[0], dev[1], slots.to(device), 245, 235)
    torch.cuda.synchronize()
    for got, want in zip(dev, expect):
        assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8))


@pytest.mark.parametrize("N,hk", [(1, 1), (4, 1), (128, 1), (1000, 1), (512, 2), (1025, 1), (1000, 2)])
def test_fused_rotation_within_tolerance(device, N, hk):
    """Writes of at most 2048 key + value vectors (N x Hk up to 1000 x 1 and
    512 x 2) take the fp32 short path, larger ones (1025 x 1, 1000 x 2) the
    MFMA one."""
    bs = 128
    pages = N // bs + 2
    k, v = synthetic.kv(N, hk, D, seed=13)
    Rk, Rv = synthetic.rotations(D, seed=17)
    slots = torch.randperm(pages * bs, generator=torch.Generator().manual_seed(2))[:N].to(torch.int64)
    slots[1::11] = -1
    caches = [torch.zeros(pages, bs, hk, D, dtype=torch.int8) for _ in range(2)]
    k_rot = orot.rotate_clip(k, Rk, 0.0)
    v_rot = orot.rotate_clip(v, Rv, 0.0)
    expect = oracle_store(k_rot, v_rot, caches, slots, 0.96, 0.92)
    dev = [c.to(device) for c in caches]
    ops = [quant.rotation_operand(R.to(device)) for R in (Rk, Rv)]
    quant.quant_write(k.to(device), v.to(device), ops[0], ops[1], dev[0], dev[1], slots.to(device),
                      245, 235, hk, D)
    torch.cuda.synchronize()
    valid = slots[slots >= 0]
    got = ostore.logical_slots(dev[0].cpu(), dev[1].cpu(), valid, hk, D)
    want = ostore.logical_slots(expect[0], expect[1], valid, hk, D)
    codes = torch.cat([got[..., 32:96], got[..., 96:160]], -1)
    codes_w = torch.cat([want[..., 32:96], want[..., 96:160]], -1)
    same = (codes == codes_w).float().mean().item()
    assert same >= 0.999, f"only {same:.5f} of code bytes match"
    kg, vg = ofmt.parse_slot_bytes(got, D)
    kw, vw = ofmt.parse_slot_bytes(want, D)
    meta_g = [ofmt.f16_from_le(got[..., 2 * j:2 * j + 1], got[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    meta_w = [ofmt.f16_from_le(want[..., 2 * j:2 * j + 1], want[..., 2 * j + 1:2 * j + 2]) for j in range(4)]
    for (a, b), (sa, sb) in (((kg, kw), (meta_g[0], meta_w[0])), ((vg, vw), (meta_g[2], meta_w[2]))):
        step = torch.maximum(sa, sb)
        assert ((a - b).abs() <= step * 1.0001 + 1e-6).all()
        assert ((sa - sb).abs() <= 2 * 2.0 ** -10 * sb.abs()).all()
    # Untouched pages stay zero: nothing written outside the valid slots.
    for c in dev:
        flat = c.cpu().view(torch.uint8).reshape(pages * bs, -1)
        mask = torch.ones(pages * bs, dtype=torch.bool)
        mask[valid] = False
        assert not flat[mask].any()


def _threshold_cases(seed: int) -> torch.Tensor:
    """Vectors that stress the clip-threshold search: Gaussian, heavy tails,
    planted ties at the usual clip ranks, values straddling bucket edges,
    few distinct values, and magnitudes spread over many octaves."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    for _ in range(16):
        rows.append(torch.randn(D, generator=g) * 1.4)
    for _ in range(8):
        rows.append(torch.empty(D).exponential_(generator=g) * torch.sign(torch.randn(D, generator=g)))
    for k in (11, 21):
        x = torch.randn(D, generator=g)
        top = x.abs().argsort(descending=True)
        x[top[k - 3:k + 3]] = x[top[k - 1]].abs() * torch.sign(x[top[k - 3:k + 3]])    # 6-way tie at rank k
        rows.append(x)
    edge = torch.randn(D, generator=g)
    a = edge.abs().max()
    # magnitudes a * 2^(-j/32) sit exactly on the buckets' edges
    edge[:64] = a * torch.pow(2.0, -torch.arange(64, dtype=torch.float32) / 32) * torch.sign(edge[:64])
    rows.append(edge)
    rows.append(torch.randint(-3, 4, (D,), generator=g).float() * 0.5)       # seven distinct values
    rows.append(torch.exp(torch.randn(D, generator=g) * 3.0) * torch.sign(torch.randn(D, generator=g)))
    rows.append(torch.cat([torch.full((20,), 50.0), torch.randn(D - 20, generator=g) * 1e-3]))
    return torch.stack(rows)


@pytest.mark.parametrize("idx", [0, 1, 64, 128, 200, 235, 240, 245, 250, 254, 255])
def test_clip_threshold_search_bit_exact(device, idx):
    """Every clip rank on adversarial vectors: bytes identical to the sort-based oracle."""
    k_rot = _threshold_cases(31).unsqueeze(1)
    v_rot = _threshold_cases(47).unsqueeze(1)
    N, hk, bs = k_rot.shape[0], 1, 16
    slots = torch.arange(N, dtype=torch.int64)
    ratio = (idx + 0.5) / D                      # clip_index(ratio) == idx
    assert quant.clip_index(ratio, D) == idx
    caches = [torch.zeros((N + bs - 1) // bs, bs, hk, D, dtype=torch.int8) for _ in range(2)]
    expect = oracle_store(k_rot, v_rot, caches, slots, ratio, ratio)
    dev = [c.to(device) for c in caches]
    quant.quant_write_prerotated(k_rot.to(device), v_rot.to(device), dev[0], dev[1], slots.to(device), idx, idx)
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(dev, expect)):
        g8, w8 = got.cpu().view(torch.uint8), want.view(torch.uint8)
        if i == 0:
            g8, w8 = zero_sign_free(g8), zero_sign_free(w8)
        bad = (g8 != w8).reshape(-1, hk * D)[:N].any(-1)
        assert not bad.any(), f"rows {bad.nonzero().flatten().tolist()} differ at idx {idx}"


@pytest.mark.parametrize("idx", [-1, 0, 64, 200, 235, 245, 255])
def test_fused_exact_rotation_bit_exact(device, idx):
    """With R a signed permutation the MFMA rotation is exact (every product
    is +-x or 0), so the fused entry must match the oracle byte for byte:
    its clip search (bucket scan, candidate ranks, exact fallback) and codes
    on the adversarial vectors above, rounded to bf16 (which adds ties), over
    4100 tokens x 2 heads (enough 32-token tiles that every workgroup walks
    several, double-buffered), with random slots and skipped ones."""
    base = torch.cat([_threshold_cases(31), _threshold_cases(47), torch.randn(64, D) * 2.0])
    N, hk, bs = 4100, 2, 64
    g = torch.Generator().manual_seed(idx + 7)
    pick = torch.randint(0, base.shape[0], (2, N * hk), generator=g)
    k = base[pick[0]].reshape(N, hk, D).to(torch.bfloat16)
    v = base[pick[1]].reshape(N, hk, D).to(torch.bfloat16)
    Rs = []
    for _ in range(2):
        perm = torch.randperm(D, generator=g)
        sign = torch.where(torch.rand(D, generator=g) < 0.5, -1.0, 1.0)
        R = torch.zeros(D, D)
        R[torch.arange(D), perm] = sign
        Rs.append(R)
    pages = (N + 40) // bs + 2
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int64)
    slots[::13] = -1
    ratio = 0.0 if idx < 0 else (idx + 0.5) / D
    assert quant.clip_index(ratio, D) == idx
    caches = make_caches(pages, bs, hk, torch.int8, seed=5)
    expect = oracle_store(k.float() @ Rs[0], v.float() @ Rs[1], caches, slots, ratio, ratio)
    dev = [c.to(device) for c in caches]
    ops = [quant.rotation_operand(R.to(device)) for R in Rs]
    quant.quant_write(k.to(device), v.to(device), ops[0], ops[1], dev[0], dev[1], slots.to(device), idx, idx, hk, D)
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(dev, expect)):
        g8, w8 = got.cpu().view(torch.uint8), want.view(torch.uint8)
        if i == 0:
            g8, w8 = zero_sign_free(g8), zero_sign_free(w8)
        bad = (g8 != w8).reshape(pages * bs, -1).any(-1)
        assert not bad.any(), f"slots {bad.nonzero().flatten()[:8].tolist()} differ at idx {idx}"


@pytest.mark.parametrize("N,hk", [(1, 1), (7, 2), (64, 2), (1024, 1)])
@pytest.mark.parametrize("idx", [-1, 0, 235, 255])
def test_short_write_exact_rotation_bit_exact(device, N, hk, idx):
    """The short path of the fused entry (at most 2048 key + value vectors,
    fp32 rotation from the operand's copy of R) with R a signed permutation:
    every rotated value is exact, so cache bytes match the oracle byte for
    byte, including skipped slots and the clip search at the edge ranks."""
    base = torch.cat([_threshold_cases(53), torch.randn(32, D) * 2.0])
    g = torch.Generator().manual_seed(1000 * N + 10 * hk + idx)
    pick = torch.randint(0, base.shape[0], (2, N * hk), generator=g)
    k = base[pick[0]].reshape(N, hk, D).to(torch.bfloat16)
    v = base[pick[1]].reshape(N, hk, D).to(torch.bfloat16)
    Rs = []
    for _ in range(2):
        perm = torch.randperm(D, generator=g)
        sign = torch.where(torch.rand(D, generator=g) < 0.5, -1.0, 1.0)
        R = torch.zeros(D, D)
        R[torch.arange(D), perm] = sign
        Rs.append(R)
    bs = 16
    pages = N // bs + 3
    slots = torch.randperm(pages * bs, generator=g)[:N].to(torch.int64)
    if N > 1:
        slots[::5] = -1
    ratio = 0.0 if idx < 0 else (idx + 0.5) / D
    caches = make_caches(pages, bs, hk, torch.int8, seed=9)
    expect = oracle_store(k.float() @ Rs[0], v.float() @ Rs[1], caches, slots, ratio, ratio)
    dev = [c.to(device) for c in caches]
    ops = [quant.rotation_operand(R.to(device)) for R in Rs]
    quant.quant_write(k.to(device), v.to(device), ops[0], ops[1], dev[0], dev[1], slots.to(device), idx, idx, hk, D)
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(dev, expect)):
        g8, w8 = got.cpu().view(torch.uint8), want.view(torch.uint8)
        if i == 0:
            g8, w8 = zero_sign_free(g8), zero_sign_free(w8)
        bad = (g8 != w8).reshape(pages * bs, -1).any(-1)
        assert not bad.any(), f"slots {bad.nonzero().flatten()[:8].tolist()} differ at idx {idx}"


def test_rotation_operand_holds_fp32_copy(device):
    """The operand's second half is R itself (fp32, row-major)."""
    R = synthetic.rotations(D, seed=3)[0]
    op = quant.rotation_operand(R.to(device)).cpu()
    assert op.numel() == 2 * 262144
    assert torch.equal(op[262144:].view(torch.float32).reshape(D, D), R.float())


@pytest.mark.parametrize("cache_dtype", [torch.int8, torch.bfloat16])
def test_short_write_geometry_and_out_of_range_slots(device, cache_dtype):
    """Short path (here 3 tokens x 4 kv heads) over int8 and bf16 cache
    geometries, with a slot beyond the cache and a skipped one: bytes match
    the oracle store everywhere (an exact rotation keeps every rotated value
    exact), so nothing outside the valid slots is written."""
    N, hk, bs, pages = 3, 4, 16, 2
    g = torch.Generator().manual_seed(77)
    base = torch.cat([_threshold_cases(59), torch.randn(16, D)])
    pick = torch.randint(0, base.shape[0], (2, N * hk), generator=g)
    k = base[pick[0]].reshape(N, hk, D).to(torch.bfloat16)
    v = base[pick[1]].reshape(N, hk, D).to(torch.bfloat16)
    Rs = []
    for _ in range(2):
        perm = torch.randperm(D, generator=g)
        sign = torch.where(torch.rand(D, generator=g) < 0.5, -1.0, 1.0)
        R = torch.zeros(D, D)
        R[torch.arange(D), perm] = sign
        Rs.append(R)
    slots = torch.tensor([5, pages * bs + 3, -1], dtype=torch.int64)
    caches = make_caches(pages, bs, hk, cache_dtype, seed=13)
    in_range = slots.clone()
    in_range[in_range >= pages * bs] = -1
    expect = oracle_store(k.float() @ Rs[0], v.float() @ Rs[1], caches, in_range, 0.96, 0.92)
    dev = [c.to(device) for c in caches]
    ops = [quant.rotation_operand(R.to(device)) for R in Rs]
    quant.quant_write(k.to(device), v.to(device), ops[0], ops[1], dev[0], dev[1], slots.to(device),
                      quant.clip_index(0.96, D), quant.clip_index(0.92, D), hk, D)
    torch.cuda.synchronize()
    for i, (got, want) in enumerate(zip(dev, expect)):
        g8, w8 = got.cpu().view(torch.uint8), want.view(torch.uint8)
        if i == 0:
            g8, w8 = zero_sign_free(g8), zero_sign_free(w8)
        assert torch.equal(g8, w8)
