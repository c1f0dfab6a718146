"""GPU parity of the MLP decode, the standalone GridEncoder and the RVQ decode.

MLP: against the oracle with the same dtype rounding (inputs, weights and
hidden activations rounded to fp16/bf16, wide accumulation), within 1e-3
absolute as stated for the fp16 MLP RGB; fp32 within 1e-5.
GridEncoder and RVQ: bit-exact.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _rand_dirs(rng, n):
    d = rng.standard_normal((n, 3)).astype(np.float32)
    return (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("C,width,dtype,N", [(16, 64, "f32", 3000), (32, 64, "f16", 3000), (64, 64, "bf16", 3000),
                                             (64, 128, "bf16", 3000), (32, 32, "f16", 3000), (64, 64, "f16", 3000),
                                             (16, 64, "bf16", 3000), (16, 32, "f16", 1000), (64, 64, "bf16", 1),
                                             (64, 64, "bf16", 63), (48, 64, "f16", 777)])
def test_mlp_rgb_decode(oracle, C, width, dtype, N):
    """Every MFMA path (16x16x32 for 16/32/64 channels at width 32/64, the
    16x16x16 one for others) and the f32 path, ragged N included."""
    from nest_splat.mlp import NestMLP
    rng = np.random.default_rng(C * 1000 + width + N)
    feat = (rng.standard_normal((N, C)) * 0.3).astype(np.float32)
    dirs = _rand_dirs(rng, N)
    m = NestMLP(C, width, dtype, seed=7).to(DEV)
    out = m.rgb_decode(torch.from_numpy(feat).to(DEV), torch.from_numpy(dirs).to(DEV)).cpu().numpy()
    ref = oracle.mlp(np.ascontiguousarray(feat.T), dirs, None, m.W1.detach().cpu().numpy(), m.W2.detach().cpu().numpy(),
                     m.W3.detach().cpu().numpy(), dtype).T
    tol = 1e-5 if dtype == "f32" else 1e-3
    np.testing.assert_allclose(out, ref, atol=tol, rtol=0)


def test_mlp_strided_features_and_mask(oracle):
    """rgb_decode on the channel-major permuted view (no copy), with the
    alpha mask and white background of the reference's render()."""
    from nest_splat.mlp import NestMLP
    from nest_splat.camera import look_at, view_ray_matrix
    rng = np.random.default_rng(3)
    C, H, W = 32, 40, 56
    color = (rng.standard_normal((C, H, W)) * 0.2).astype(np.float32)
    alpha = rng.uniform(0, 1, (H, W)).astype(np.float32)
    alpha[rng.uniform(size=(H, W)) < 0.3] = 0.0
    m = NestMLP(C, 64, "f16", seed=11).to(DEV)
    cam = look_at((0.3, -3, 1.0), (0, 0, 0), 50.0, W, H)
    ct = torch.from_numpy(color).to(DEV)
    feat_view = ct.view(C, -1).permute(1, 0)
    assert not feat_view.is_contiguous()
    bg = np.array([1.0, 1.0, 1.0], np.float32)
    img = m.decode_image(ct, view_ray_matrix(cam), alpha=torch.from_numpy(alpha).to(DEV),
                         bg=torch.from_numpy(bg)).cpu().numpy()
    dirs = oracle.ray_dirs(cam)
    ref = oracle.mlp(color.reshape(C, -1), dirs, alpha.reshape(-1), m.W1.detach().cpu().numpy(),
                     m.W2.detach().cpu().numpy(), m.W3.detach().cpu().numpy(), "f16", bg).reshape(3, H, W)
    np.testing.assert_allclose(img, ref, atol=1e-3, rtol=0)
    # masked pixels are exactly the background
    np.testing.assert_array_equal(img[:, alpha == 0], np.broadcast_to(bg[:, None], (3, int((alpha == 0).sum()))))
    out = m.rgb_decode(feat_view, torch.from_numpy(dirs).to(DEV)).cpu().numpy()
    ref2 = oracle.mlp(color.reshape(C, -1), dirs, None, m.W1.detach().cpu().numpy(), m.W2.detach().cpu().numpy(),
                      m.W3.detach().cpu().numpy(), "f16").T
    np.testing.assert_allclose(out, ref2, atol=1e-3, rtol=0)


@pytest.mark.parametrize("L,F,log2T,half,B", [(8, 2, 14, False, 5000), (16, 4, 16, False, 5000), (16, 2, 15, True, 5000),
                                              (4, 8, 12, False, 5000), (6, 1, 10, False, 5000), (16, 4, 16, True, 5000),
                                              (16, 4, 19, False, 300_001)])
def test_grid_encode_parity(oracle, L, F, log2T, half, B):
    """Bit-exact against the oracle: binary32 tables of the common level
    layout take the level-per-wave kernel (300,001 points: more 64-point
    blocks than workgroups, a ragged last block), binary16 the generic one."""
    from gridencoder import GridEncoder
    rng = np.random.default_rng(L * 100 + F)
    enc = GridEncoder(3, L, F, 1.5, 16, log2T).to(DEV)
    tab = rng.uniform(-0.1, 0.1, enc.embeddings.shape).astype(np.float32)
    if half:
        tab = tab.astype(np.float16)
    with torch.no_grad():
        enc.embeddings = torch.nn.Parameter(torch.from_numpy(tab).to(DEV), requires_grad=False)
    x = rng.uniform(-0.05, 1.05, (B, 3)).astype(np.float32)
    x[:7] = [[0, 0, 0], [1, 1, 1], [0.5, 0.5, 0.5], [1, 0, 1], [0, 1, 0.25], [1.0, 1.0, 0.999], [0.0, 0.0, 1e-7]]
    out = enc(torch.from_numpy(x).to(DEV)).float().cpu().numpy()
    grid = oracle.make_grid(L, F, float(np.log2(1.5)), 16, enc._offsets_host, tab, (0.0, 1.0))
    ref = oracle.grid_encode(grid, x)
    np.testing.assert_array_equal(out, ref)


def grid_encode_np(x, table, offsets, L, F, S, H, gridtype, align):
    """Brute-force restatement of kernel_grid (gridencoder.cu:87-242) for any D,
    float32 table, used to pin D != 3 and the tiled grid type."""
    B, D = x.shape
    primes = [1, 2654435761, 805459861, 3674653429, 2097192037]
    out = np.zeros((B, L * F), np.float32)
    for b in range(B):
        u = x[b]
        if np.any(u < 0) or np.any(u > 1):
            continue
        for l in range(L):
            hs = int(offsets[l + 1] - offsets[l])
            scale = np.float32(np.float32(np.exp2(np.float64(np.float32(l) * np.float32(S)))) * np.float32(H)) - np.float32(1)
            res = int(np.ceil(scale)) + 1
            pos = (u * scale + np.float32(0 if align else 0.5)).astype(np.float32)
            g = np.floor(pos).astype(np.int64)
            pos = (pos - g.astype(np.float32)).astype(np.float32)
            acc = np.zeros(F, np.float32)
            for c in range(1 << D):
                w = np.float32(1)
                q = []
                for d in range(D):
                    if c & (1 << d):
                        w = np.float32(w * pos[d]); q.append(int(g[d]) + 1)
                    else:
                        w = np.float32(w * np.float32(1 - pos[d])); q.append(int(g[d]))
                stride, idx = 1, 0
                for d in range(D):
                    if stride > hs:
                        break
                    idx = (idx + q[d] * stride) & 0xFFFFFFFF
                    stride = (stride * (res if align else res + 1)) & 0xFFFFFFFF
                if gridtype == 0 and stride > hs:
                    idx = 0
                    for d in range(D):
                        idx ^= (q[d] * primes[d]) & 0xFFFFFFFF
                idx = idx % hs
                acc = (acc + w * table[offsets[l] + idx]).astype(np.float32)
            out[b, l * F:(l + 1) * F] = acc
    return out


@pytest.mark.parametrize("D,gridtype,align", [(2, 0, False), (4, 0, False), (3, 1, False), (3, 0, True), (5, 1, True)])
def test_grid_encode_dims_and_types(D, gridtype, align):
    from gridencoder import GridEncoder
    rng = np.random.default_rng(D * 10 + gridtype)
    L, F = 5, 2
    enc = GridEncoder(D, L, F, 1.7, 8, 10, gridtype="tiled" if gridtype else "hash", align_corners=align).to(DEV)
    tab = rng.uniform(-1, 1, enc.embeddings.shape).astype(np.float32)
    with torch.no_grad():
        enc.embeddings = torch.nn.Parameter(torch.from_numpy(tab).to(DEV), requires_grad=False)
    x = rng.uniform(0, 1, (300, D)).astype(np.float32)
    out = enc(torch.from_numpy(x).to(DEV)).cpu().numpy()
    ref = grid_encode_np(x, tab, enc._offsets_host, L, F, float(np.log2(1.7)), 8, gridtype, align)
    np.testing.assert_allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_rvq_decode_bit_exact(oracle):
    from nest_splat.rvq import RVQAttributes
    from nest_splat.scene import RVQ_BIAS
    rng = np.random.default_rng(5)
    P, S, K = 50_000, 4, 4096
    cbs = {a: (0.1 * rng.standard_normal((S, K, d))).astype(np.float32) for a, d in (("scale", 2), ("rotation", 4), ("opacity", 1))}
    idxs = {a: rng.integers(0, K, (P, S)).astype(np.uint16) for a in cbs}
    idxs["scale"][:3] = [[0, 0, 0, 0], [K - 1] * 4, [1, 2, 3, 4]]
    rv = RVQAttributes.from_numpy(cbs, idxs, RVQ_BIAS, DEV)
    dec = rv.decode(raw=True)
    raw = {a: oracle.rvq_decode(cbs[a], idxs[a], RVQ_BIAS[a]) for a in cbs}
    for a in cbs:
        np.testing.assert_array_equal(dec[a + "_raw"].cpu().numpy(), raw[a])
    sc, rot, op = oracle.activate(raw["scale"], raw["rotation"], raw["opacity"])
    np.testing.assert_array_equal(dec["scale"].cpu().numpy(), sc)
    np.testing.assert_array_equal(dec["rotation"].cpu().numpy(), rot)
    np.testing.assert_array_equal(dec["opacity"].cpu().numpy()[:, 0], op)


@pytest.mark.parametrize("P,K_scale,K_rot,K_op", [(1_000_003, 4096, 4096, 4096), (300_001, 4096, 1024, 512),
                                                   (2_047, 4096, 4096, 4096)])
def test_rvq_batch_fused_bit_exact(oracle, P, K_scale, K_rot, K_op):
    """The fused persistent batch decode: ragged P; at 1M splats each
    workgroup decodes several chunks, so the rotation codebook (4096 x 4,
    held one stage pair at a time) is gathered in both pair orders, while
    the scale and opacity codebooks stay resident; a 1024-entry rotation
    codebook is resident too.  Raw sums and activations against the oracle's
    ordered float32 sum, an out-of-range index per attribute decoding to NaN."""
    from nest_splat.rvq import RVQAttributes
    from nest_splat.scene import RVQ_BIAS
    rng = np.random.default_rng(P)
    S = 4
    dims = {"scale": (2, K_scale), "rotation": (4, K_rot), "opacity": (1, K_op)}
    cbs = {a: (0.1 * rng.standard_normal((S, K, d))).astype(np.float32) for a, (d, K) in dims.items()}
    idxs = {a: rng.integers(0, K, (P, S)).astype(np.uint16) for a, (d, K) in dims.items()}
    badrow = {"scale": P // 3, "rotation": P - 1, "opacity": 1}
    for a, (d, K) in dims.items():
        idxs[a][0] = K - 1
        idxs[a][badrow[a], a == "rotation" and 3 or 1] = K
    dec = RVQAttributes.from_numpy(cbs, idxs, RVQ_BIAS, DEV).decode(raw=True)
    torch.cuda.synchronize()
    for a, (d, K) in dims.items():
        got = dec[a + "_raw"].cpu().numpy()
        assert np.isnan(got[badrow[a]]).all()
        good = np.ones(P, bool)
        good[badrow[a]] = False
        ref = oracle.rvq_decode(cbs[a], np.where(good[:, None], idxs[a], 0).astype(np.uint16), RVQ_BIAS[a])
        np.testing.assert_array_equal(got[good], ref[good])
        act = dec[a].cpu().numpy()
        assert np.isnan(act[badrow[a]]).all()
    raw = {a: np.where(np.isnan(dec[a + "_raw"].cpu().numpy()), 0, dec[a + "_raw"].cpu().numpy()) for a in dims}
    sc, rot, op = oracle.activate(raw["scale"], raw["rotation"], raw["opacity"])
    keep = np.ones(P, bool)
    keep[list(badrow.values())] = False
    np.testing.assert_array_equal(dec["scale"].cpu().numpy()[keep], sc[keep])
    np.testing.assert_array_equal(dec["rotation"].cpu().numpy()[keep], rot[keep])
    np.testing.assert_array_equal(dec["opacity"].cpu().numpy()[keep, 0], op[keep])


def test_rvq_out_of_range_index_is_nan():
    from nest_splat.rvq import rvq_decode
    cb = torch.zeros((2, 8, 2), dtype=torch.float32, device=DEV)
    idx = torch.tensor([[0, 1], [9, 0], [7, 7]], dtype=torch.int16, device=DEV)
    out = rvq_decode(cb, idx).cpu().numpy()
    assert np.isnan(out[1]).all() and not np.isnan(out[0]).any() and not np.isnan(out[2]).any()


@pytest.mark.parametrize("P,S,K,dim", [(70_001, 4, 4096, 4), (9_999, 4, 4096, 2), (1_000, 4, 512, 1),
                                       (33_333, 3, 1024, 4), (5_000, 4, 2048, 3), (20_000, 4, 65536, 2)])
def test_rvq_decode_paths_bit_exact(oracle, P, S, K, dim):
    """Both decode kernels: the LDS-staged one (4 stages, a stage codebook of
    at most 64 KiB, dim 1, 2 or 4) and the gather one (other shapes), with
    ragged P, against the oracle's ordered float32 sum; an out-of-range index
    in either decodes to NaN."""
    from nest_splat.rvq import rvq_decode
    rng = np.random.default_rng(P + K)
    cb = (0.1 * rng.standard_normal((S, K, dim))).astype(np.float32)
    idx = rng.integers(0, K, (P, S)).astype(np.uint16)
    idx[0] = K - 1
    bad = K < 65536
    if bad:
        idx[P // 2, S - 1] = K  # one past the codebook
    bias = rng.standard_normal(dim).astype(np.float32)
    out = rvq_decode(torch.from_numpy(cb).to(DEV), torch.from_numpy(idx.view(np.int16)).to(DEV), bias=bias).cpu().numpy()
    good = np.ones(P, bool)
    if bad:
        good[P // 2] = False
        assert np.isnan(out[P // 2]).all()
    ref = oracle.rvq_decode(cb, np.where(good[:, None], idx, 0).astype(np.uint16), bias)
    np.testing.assert_array_equal(out[good], ref[good])


@pytest.mark.parametrize("C,width,dtype", [(16, 64, "bf16"), (32, 32, "f16"), (64, 64, "bf16"), (64, 32, "f16"),
                                           (64, 128, "bf16"), (64, 128, "f16")])
def test_mlp_decode_image_blocks(oracle, C, width, dtype):
    """decode_image on the render's contiguous [C, H, W] map (the 256-pixel
    block kernel: 4 waves for widths 32 and 64, 8 for width 128; a partial
    last block), with a mask and white background, against the oracle."""
    from nest_splat.camera import look_at, view_ray_matrix
    from nest_splat.mlp import NestMLP
    rng = np.random.default_rng(C + width)
    H, W = 24, 37  # 888 pixels: three full blocks and a partial one
    color = (rng.standard_normal((C, H, W)) * 0.25).astype(np.float32)
    alpha = rng.uniform(0, 1, (H, W)).astype(np.float32)
    alpha[rng.uniform(size=(H, W)) < 0.2] = 0.0
    m = NestMLP(C, width, dtype, seed=C).to(DEV)
    cam = look_at((0.5, -3, 0.8), (0, 0, 0), 55.0, W, H)
    bg = np.array([1.0, 1.0, 1.0], np.float32)
    img = m.decode_image(torch.from_numpy(color).to(DEV), view_ray_matrix(cam), alpha=torch.from_numpy(alpha).to(DEV),
                         bg=torch.from_numpy(bg)).cpu().numpy()
    ref = oracle.mlp(color.reshape(C, -1), oracle.ray_dirs(cam), alpha.reshape(-1), m.W1.detach().cpu().numpy(),
                     m.W2.detach().cpu().numpy(), m.W3.detach().cpu().numpy(), dtype, bg).reshape(3, H, W)
    np.testing.assert_allclose(img, ref, atol=1e-3, rtol=0)
