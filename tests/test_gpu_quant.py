"""GPU parity of the quantizers (fp8.py:39-47, fp8.py:68) against the CPU oracle.

Bar: e4m3fn bytes and fp32 scales bit-exact (NaN scales compare as NaN).
"""
import numpy as np
import pytest
import torch

import fp8
from helpers import bf16_bits, f32_bits, same_scales, to_dev, u8
from oracle import bf16 as ob
from oracle import cbind, fp8_ref

pytestmark = pytest.mark.gpu


def _special_rows(rng, K):
    """Rows exercising the edge cases of fp8.py:42-46."""
    rows = []
    rows.append(np.zeros(K, np.float32))                                  # all zero -> s = 1e-30
    r = np.zeros(K, np.float32); r[::2] = -0.0; rows.append(r)            # -0 -> 0x80
    rows.append(np.ones(K, np.float32))                                   # ones KAT
    r = rng.standard_normal(K).astype(np.float32); r[5] = np.nan; rows.append(r)      # NaN block
    r = rng.standard_normal(K).astype(np.float32); r[7] = np.inf; rows.append(r)      # +inf block
    r = rng.standard_normal(K).astype(np.float32); r[9] = -np.inf; r[10] = np.inf; rows.append(r)
    r = (rng.standard_normal(K) * 1e-38).astype(np.float32); rows.append(r)           # subnormal-ish
    r = (rng.standard_normal(K) * 1e-30).astype(np.float32); rows.append(r)           # scale floor
    r = (rng.standard_normal(K) * 3e38).astype(np.float32); rows.append(r)            # near max
    r = np.full(K, 2.0 ** -133, np.float32); r[0] = 1.0; rows.append(r)               # bf16 min subnormal
    return ob.f32_to_bf16(np.stack(rows))


def _check_rows(x_u16, dev):
    q, s = fp8.quantize_fp8(to_dev(x_u16, dev))
    qo, so = fp8_ref.quantize_fp8(ob.bf16_to_f32(x_u16))
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("shape", [(1, 128), (3, 384), (17, 256), (2048, 768), (130, 2304)])
def test_quantize_rows_random(dev, shape):
    rng = np.random.default_rng(hash(shape) % 2**32)
    x = ob.randn_bf16(rng, shape)
    x[..., 3] = ob.f32_to_bf16(np.float32(60.0))            # outlier in the first block
    _check_rows(x, dev)


def test_quantize_rows_special_values(dev):
    rng = np.random.default_rng(7)
    _check_rows(_special_rows(rng, 256), dev)


def test_quantize_rows_every_bf16_value(dev):
    """All 65536 bf16 patterns, grouped 128 per block in several orders."""
    allv = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    rng = np.random.default_rng(11)
    for perm in (allv, rng.permutation(allv), np.sort(allv)[::-1].copy()):
        _check_rows(perm.reshape(-1, 128), dev)


def test_quantize_rows_f32_input(dev):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 512)) * np.exp(rng.standard_normal((64, 512)))).astype(np.float32)
    x[0, :128] = 0.0
    q, s = fp8.quantize_fp8(torch.from_numpy(x).to(dev))
    qo, so = fp8_ref.quantize_fp8(x)
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


@pytest.mark.parametrize("shape", [(128, 8), (256, 72), (768, 3072), (384, 200)])
def test_quantize_cols_transposed(dev, shape):
    """fp8.py:68: quantize b.T of b (K, N) along K."""
    rng = np.random.default_rng(sum(shape))
    b = ob.randn_bf16(rng, shape, std=0.02)
    q, s = fp8.quantize_fp8(to_dev(b, dev), transpose=True)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(b).T))
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


def test_quantize_cols_special_values(dev):
    rng = np.random.default_rng(5)
    b = np.ascontiguousarray(_special_rows(rng, 128).T)           # (128, 10) -> pad cols to 16
    b = np.concatenate([b, ob.randn_bf16(rng, (128, 6))], axis=1)
    q, s = fp8.quantize_fp8(to_dev(b, dev), transpose=True)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(b).T))
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)


def test_quantize_full_size_c3_operands(dev):
    """C3 operands at full size, checked against the C oracle."""
    rng = np.random.default_rng(2)
    x = ob.randn_bf16(rng, (8192, 2048))
    w = ob.randn_bf16(rng, (2048, 8192), std=0.02)
    qx, sx = fp8.quantize_fp8(to_dev(x, dev))
    qo, so = cbind.quantize_rows_bf16(x)
    np.testing.assert_array_equal(u8(qx), qo)
    np.testing.assert_array_equal(f32_bits(sx), so.view(np.uint32))
    qw, sw = fp8.quantize_fp8(to_dev(w, dev), transpose=True)
    qo, so = cbind.quantize_cols_bf16(w)
    np.testing.assert_array_equal(u8(qw), qo)
    np.testing.assert_array_equal(f32_bits(sw), so.view(np.uint32))


@pytest.mark.parametrize("shape", [(128, 128), (256, 384), (1024, 640), (4096, 4096), (8192, 8192),
                                   (16384, 4096), (2048, 32768)])
def test_quantize_dual_equals_separate(dev, shape):
    """tg_quantize_dual = tg_quantize_rows + tg_quantize_cols, bit for bit (C3's dY at full size;
    8192^2, 16384 x 4096 and 2048 x 32768 take the XCD-blocked tile order)."""
    rng = np.random.default_rng(sum(shape) + 3)
    x = to_dev(ob.randn_bf16(rng, shape, std=1e-3), dev)
    q, s, qt, st = fp8.quantize_fp8_dual(x)
    q1, s1 = fp8.quantize_fp8(x)
    q2, s2 = fp8.quantize_fp8(x, transpose=True)
    assert torch.equal(q.view(torch.uint8), q1.view(torch.uint8))
    assert torch.equal(qt.view(torch.uint8), q2.view(torch.uint8))
    assert np.array_equal(f32_bits(s), f32_bits(s1)) and np.array_equal(f32_bits(st), f32_bits(s2))


@pytest.mark.parametrize("shapes", [((8192, 2048), (2048, 8192)),     # C3's x and W
                                    ((384, 256), (8192, 8192)),      # job 1 at slot 6: identity order
                                    ((1024, 1024), (8192, 8192)),    # job 1 at slot 64: XCD-blocked
                                    ((128, 128), (256, 640))])
def test_quantize_dual_pair_equals_dual(dev, shapes):
    """tg_quantize_dual_pair = tg_quantize_dual on each tensor, bit for bit, with
    the special-value rows of the oracle test planted in both tensors."""
    rng = np.random.default_rng(sum(map(sum, shapes)))
    xs = []
    for shape in shapes:
        x = ob.randn_bf16(rng, shape, std=0.02)
        k = min(256, shape[1])
        x[:10, :k] = _special_rows(rng, k)
        xs.append(to_dev(x, dev))
    pair = fp8.quantize_fp8_dual_pair(xs[0], xs[1])
    for x, got in zip(xs, pair):
        want = fp8.quantize_fp8_dual(x)
        for g, w in zip(got, want):
            if g.dtype == torch.float32:
                assert np.array_equal(f32_bits(g), f32_bits(w))
            else:
                assert torch.equal(g.view(torch.uint8), w.view(torch.uint8))


@pytest.mark.parametrize("shape", [(128, 128), (256, 384), (1024, 640), (8192, 8192), (16384, 4096)])
def test_quantize_dual_km_is_the_transposed_scale_layout(dev, shape):
    """tg_quantize_dual_km: the bytes of tg_quantize_dual, every scale array
    stored K-block-major (scales_km[kb, r] == scales[r, kb]), bit for bit, with
    special-value rows planted (NaN / inf scales land in the right slot)."""
    rng = np.random.default_rng(sum(shape) + 21)
    x = ob.randn_bf16(rng, shape, std=0.02)
    x[:10, :128] = _special_rows(rng, 128)
    xd = to_dev(x, dev)
    q, s, qt, st = fp8.quantize_fp8_dual(xd)
    kq, ks, kqt, kst = fp8._quantize_dual_km(xd, 128)
    assert ks.shape == (shape[1] // 128, shape[0]) and kst.shape == (shape[0] // 128, shape[1])
    assert torch.equal(kq, q.view(torch.uint8)) and torch.equal(kqt, qt.view(torch.uint8))
    assert np.array_equal(f32_bits(ks), f32_bits(s).T) and np.array_equal(f32_bits(kst), f32_bits(st).T)


@pytest.mark.parametrize("shapes", [((8192, 2048), (2048, 8192)), ((384, 256), (1024, 640))])
def test_quantize_dual_pair_km(dev, shapes):
    """tg_quantize_dual_pair_km = tg_quantize_dual_km on each tensor, bit for bit."""
    rng = np.random.default_rng(sum(map(sum, shapes)) + 5)
    xs = [to_dev(ob.randn_bf16(rng, s, std=0.02), dev) for s in shapes]
    pair = fp8._quantize_dual_pair_km(xs[0], xs[1], 128)
    for x, got in zip(xs, pair):
        want = fp8._quantize_dual_km(x, 128)
        for g, w in zip(got, want):
            assert np.array_equal(f32_bits(g), f32_bits(w)) if g.dtype == torch.float32 else torch.equal(g, w)


def test_quantize_dual_pair_skips_empty(dev):
    """A tensor with no rows is skipped (null pointers allowed); the other is quantized."""
    import _tglib as L
    rng = np.random.default_rng(12)
    x = to_dev(ob.randn_bf16(rng, (256, 384)), dev)
    q = torch.empty((256, 384), dtype=torch.uint8, device=dev)
    s = torch.empty((256, 3), dtype=torch.float32, device=dev)
    qt = torch.empty((384, 256), dtype=torch.uint8, device=dev)
    st = torch.empty((384, 2), dtype=torch.float32, device=dev)
    P = L.ptr
    L.check(L.lib().tg_quantize_dual_pair(None, 0, 384, None, None, None, None, P(x), 256, 384, P(q),
                                          P(s), P(qt), P(st), 128, L.stream_of(x)))
    want = fp8.quantize_fp8_dual(x)
    assert torch.equal(q, want[0].view(torch.uint8)) and torch.equal(qt, want[2].view(torch.uint8))
    assert np.array_equal(f32_bits(s), f32_bits(want[1])) and np.array_equal(f32_bits(st), f32_bits(want[3]))
    with pytest.raises(ValueError, match="multiples of 128"):
        L.check(L.lib().tg_quantize_dual_pair(P(x), 256, 384, P(q), P(s), P(qt), P(st), P(x), 200, 384,
                                              P(q), P(s), P(qt), P(st), 128, L.stream_of(x)))


def test_quantize_dual_special_values(dev):
    """Edge-case blocks in both directions against the oracle."""
    rng = np.random.default_rng(6)
    rows = _special_rows(rng, 256)                                 # (10, 256)
    x = np.concatenate([rows, ob.randn_bf16(rng, (118, 256))], axis=0)
    x[20:30, :128] = _special_rows(rng, 128)                      # special row blocks mid-tile
    cols = np.ascontiguousarray(_special_rows(rng, 128).T)         # (128, 10): special columns
    x[:, 200:210] = cols
    q, s, qt, st = fp8.quantize_fp8_dual(to_dev(x, dev))
    qo, so = fp8_ref.quantize_fp8(ob.bf16_to_f32(x))
    np.testing.assert_array_equal(u8(q), qo)
    assert same_scales(s.cpu().numpy(), so)
    qo, so = fp8_ref.quantize_fp8(np.ascontiguousarray(ob.bf16_to_f32(x).T))
    np.testing.assert_array_equal(u8(qt), qo)
    assert same_scales(st.cpu().numpy(), so)


def test_quantize_deterministic(dev):
    rng = np.random.default_rng(9)
    x = to_dev(ob.randn_bf16(rng, (512, 1024)), dev)
    q1, s1 = fp8.quantize_fp8(x)
    q2, s2 = fp8.quantize_fp8(x)
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(s1, s2)


@pytest.mark.parametrize("K,N", [(512, 300), (256, 384)])
def test_weight_128x128(dev, K, N):
    """Both load paths of the tile quantizer: element loads (N % 8 != 0) and
    16-byte loads, with a NaN tile, an inf tile and an all-zero tile."""
    rng = np.random.default_rng(4 + N)
    w = ob.randn_bf16(rng, (K, N), std=0.02)
    w[3, 5] = 0x7FC0                         # NaN in tile (0, 0)
    w[130, 200] = 0xFF80                     # -inf in tile (1, 1)
    w[128:256, 256:] = 0                     # tile (1, 2): all zero (scale floor)
    wq, ws, bn = fp8.quantize_weight(to_dev(w, dev), layout="128x128")
    assert bn == 128
    qo, so = fp8_ref.quantize_weight_128x128(np.ascontiguousarray(ob.bf16_to_f32(w).T))
    np.testing.assert_array_equal(u8(wq), qo)
    np.testing.assert_array_equal(f32_bits(ws), so.view(np.uint32))


def test_errors(dev):
    x = torch.zeros((4, 200), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError, match="not divisible by block_k"):
        fp8.quantize_fp8(x)
    with pytest.raises(NotImplementedError):   # the fused dual quantizer is block_k = 128 only
        fp8.quantize_fp8_dual(torch.zeros((256, 256), dtype=torch.bfloat16, device=dev), block_k=64)
    q, s = fp8.quantize_fp8(torch.zeros((0, 256), dtype=torch.bfloat16, device=dev))
    assert q.shape == (0, 256) and s.shape == (0, 2)
    assert bf16_bits is not None


@pytest.mark.parametrize("shape", [(1, 9216), (8, 9216), (3, 256), (64, 1024)])
def test_quantize_relu2_bit_exact(dev, shape):
    """tg_quantize_rows_relu2: the oracle's _quantize_to_fp8 of bf16(relu(x)^2)
    (model.py:72 on bf16 values: relu exact, the square rounded once)."""
    import fp8
    rng = np.random.default_rng(sum(shape))
    x = ob.randn_bf16(rng, shape, std=3.0)
    x[0, :3] = [0x7FC0, 0x8000, 0xFF80]        # NaN, -0, -inf
    q, s = fp8.quantize_relu2(to_dev(x, dev))
    xf = ob.bf16_to_f32(x)
    with np.errstate(invalid="ignore"):
        r = np.where(np.isnan(xf), xf, np.maximum(xf, np.float32(0)))
    u = ob.round_bf16((r * r).astype(np.float32))
    q_o, s_o = fp8_ref.quantize_fp8(u)
    np.testing.assert_array_equal(u8(q), q_o)
    assert same_scales(s.cpu().numpy(), s_o)
