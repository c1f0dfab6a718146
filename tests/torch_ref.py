"""Independent float64 torch forward of the render (mode 0) and its inputs,
used to pin the backward oracle by automatic differentiation.

TEST INFRASTRUCTURE ONLY.  The discrete decisions of the forward (which
tile/splat pairs are accepted, the rho3d/rho2d branch, the per-pixel cut-off
where T (1 - alpha) falls below 1e-4, the median contributor (the last hit
taken while T > 0.5), the hash-grid cell of every corner) are taken from
float32 replicas of the forward's rules, with the oracle's exp; the cut-off
and median are checked against the oracle's n_contrib.  Everything
continuous is evaluated in float64 torch, so autograd gives the exact
derivative of the forward the oracle computes.  The gradients the reference defines differently from that
derivative are handled as the reference does: the 0.99 alpha clamp is
differentiated as if absent (straight-through), with beta > 0 the position
terms carry the activated G' in place of the raw g, the auxiliary outputs
7..13 carry no gradient.
"""
from __future__ import annotations

import numpy as np
import torch

NEAR, FAR = 0.2, 100.0
f32 = np.float32


def level_scale(O, S, H, l):
    import ctypes as ct
    sc = ct.c_float()
    res = ct.c_uint32()
    O.lib().or_level_scale(float(S), int(H), int(l), ct.byref(sc), ct.byref(res))
    return np.float32(sc.value), int(res.value)


def grid_index(align, hsize, res, g):
    """get_grid_index + fast_hash (CR/hashgrid.h:7-40) on uint64 arrays [..., 3]."""
    g = g.astype(np.uint64)
    stride, index = 1, np.zeros(g.shape[:-1], np.uint64)
    r1 = res if align else res + 1
    d = 0
    while d < 3 and stride <= hsize:
        index = (index + g[..., d] * np.uint64(stride)) & np.uint64(0xFFFFFFFF)
        stride *= r1
        d += 1
    if stride > hsize:
        m = np.uint64(0xFFFFFFFF)
        index = (g[..., 0] & m) ^ ((g[..., 1] * np.uint64(2654435761)) & m) ^ ((g[..., 2] * np.uint64(805459861)) & m)
    return (index % np.uint64(hsize)).astype(np.int64)


def _pair_decisions(O, Tm, xy, opa, px, py, beta, kernel_type=0, shp=None):
    """float32 replica of the per-pair acceptance (CR/forward.cu:834-921):
    returns accepted, use3d, the float32 s (for the cells) and alpha.
    kernel_type 1-3 take the per-splat shapes shp (CR/forward.cu:864-900)."""
    Tu, Tv, Tw = Tm[..., 0:3], Tm[..., 3:6], Tm[..., 6:9]
    k = px[..., None] * Tw - Tu
    l = py[..., None] * Tw - Tv
    p0 = k[..., 1] * l[..., 2] - k[..., 2] * l[..., 1]
    p1 = k[..., 2] * l[..., 0] - k[..., 0] * l[..., 2]
    p2 = k[..., 0] * l[..., 1] - k[..., 1] * l[..., 0]
    with np.errstate(divide="ignore", invalid="ignore"):
        sx, sy = p0 / p2, p1 / p2
    rho3d = sx * sx + sy * sy
    dx, dy = xy[..., 0] - px, xy[..., 1] - py
    rho2d = f32(2.0) * (dx * dx + dy * dy)
    use3d = rho3d <= rho2d
    rho = np.minimum(rho3d, rho2d)
    depth = np.where(use3d, (sx * Tw[..., 0] + sy * Tw[..., 1]) + Tw[..., 2], Tw[..., 2])
    with np.errstate(over="ignore", invalid="ignore", divide="ignore"):
        ok = f32(-0.5) * rho <= 0
        if kernel_type == 1:
            ok = rho < f32(1)
            G = O.powf(np.where(ok, f32(1) - rho, f32(0.5)), shp)
        elif kernel_type == 2:
            g = O.expf(f32(-0.5) * rho)
            b = np.broadcast_to(shp, g.shape).astype(f32)
            G = np.where(b > 0, (f32(1) + b) * g / (f32(1) + b * g), g).astype(f32)
        elif kernel_type == 3:
            pt = O.powf(np.maximum(rho, f32(1e-8)), f32(0.5) * shp)
            ok = f32(-0.5) * pt <= 0
            G = O.expf(f32(-0.5) * pt)
        else:
            G = O.expf(f32(-0.5) * rho)
            if beta > 0:
                G = ((1.0 + beta) * G.astype(np.float64) / (1.0 + (f32(beta) * G).astype(np.float64))).astype(f32)
        alpha = np.minimum(f32(0.99), opa * G)
    acc = (p2 != 0) & (depth >= f32(NEAR)) & ok & (alpha >= f32(1.0 / 255.0))
    return acc, use3d, sx, sy, alpha


def _pixel_cutoff(acc, alpha):
    """Front-to-back float32 transmittance per pixel (rows): a hit whose
    T (1 - alpha) < 1e-4 ends the pixel uncounted; the median is the last hit
    taken while T > 0.5 (CR/forward.cu:894-930, :1917-1920).  Returns the hits
    taken [npix, n], the last contributor and the median contributor
    (1-based positions in the tile's list, 0 for none)."""
    npix, n = acc.shape
    T = np.ones(npix, f32)
    done = np.zeros(npix, bool)
    take = np.zeros_like(acc)
    last = np.zeros(npix, np.int64)
    med = np.zeros(npix, np.int64)
    for j in range(n):
        ok = acc[:, j] & ~done
        tT = (T * (f32(1) - alpha[:, j])).astype(f32)
        stop = ok & (tT < f32(1e-4))
        done |= stop
        t = ok & ~stop
        med = np.where(t & (T > f32(0.5)), j + 1, med)
        last = np.where(t, j + 1, last)
        take[:, j] = t
        T = np.where(t, tT, T)
    return take, last, med


def _kernel_g(kernel_type, rho, shp, beta):
    """G of kernel_type 1-3 in float64 with the gradients the reference's
    backward gives it (CR/backward.cu:1864-1909, :1963-2039): the beta
    kernel's position term is half the derivative (dG/drho where the other
    kernels use 2 dG/drho), its shape term G ln(1 - rho); a flex splat
    without its own beta (<= 0) has G = g with the position gradient scaled
    by 1 + beta of the settings when that is > 0; flex with beta > 0 and the
    general kernel are exact derivatives."""
    if kernel_type == 1:
        rho_h = rho.detach() + 0.5 * (rho - rho.detach())
        return torch.clamp_min(1.0 - rho_h, 1e-30) ** shp
    if kernel_type == 2:
        g = torch.exp(-0.5 * rho)
        on = shp > 0
        if beta > 0:
            g_pos = g.detach() + (g - g.detach()) * (1.0 + beta)
        else:
            g_pos = g
        bsafe = torch.where(on, shp, torch.zeros_like(shp))
        return torch.where(on, (1.0 + bsafe) * g / (1.0 + bsafe * g), g_pos)
    pt = torch.clamp_min(rho, 1e-8) ** (0.5 * shp)
    return torch.exp(-0.5 * pt)


def render_forward(O, pre, binres, fwd, W, H, C, leaves, grid=None, beta=0.0, homotrans_np=None, ap_level=None,
                   kernel_type=0):
    """Differentiable forward of out_color [C,H,W] and allmap channels 0..6.

    leaves: dict of float64 tensors with requires_grad: T [P,9], xy [P,2],
    normal [P,3], opacity [P], and colors [P,C] (colour path) or homo [P,16]
    and table [rows,F] (hash path), with rows [P,R] ahead of the grid
    features in render mode 4, or rows [P,total*F+1] blended with them in
    render mode 12 (grid["hyb12"] = per-splat levels).  grid: dict(L, F, S, H, offsets, vmin,
    vmax) for the hash path (non-contracted, not align_corners, linear).
    kernel_type 1-3 take leaves["shape"] [P]."""
    HW = W * H
    gx = (W + 15) // 16
    ranges = binres["ranges"].reshape(-1, 2)
    vals = binres["vals"]
    ncon = fwd["n_contrib"].reshape(2, HW)
    color = torch.zeros((C, HW), dtype=torch.float64)
    others = torch.zeros((7, HW), dtype=torch.float64)
    Tm32, xy32, no32 = pre["transmat"], pre["xy"], pre["normal_opacity"]
    for tile in range(ranges.shape[0]):
        r0, r1 = int(ranges[tile, 0]), int(ranges[tile, 1])
        if r1 <= r0:
            continue
        ty, tx = divmod(tile, gx)
        yy, xx = np.meshgrid(np.arange(16), np.arange(16), indexing="ij")
        px = (tx * 16 + xx).reshape(-1)
        py = (ty * 16 + yy).reshape(-1)
        inside = (px < W) & (py < H)
        px, py = px[inside], py[inside]
        pid = py * W + px
        ids = vals[r0:r1].astype(np.int64)
        n = ids.shape[0]
        shp32 = None if kernel_type == 0 else leaves["shape"].detach().numpy().astype(f32)[ids][None]
        acc, use3d, sx32, sy32, a32 = _pair_decisions(O, Tm32[ids][None], xy32[ids][None], no32[ids, 3][None],
                                                      px.astype(f32)[:, None], py.astype(f32)[:, None], beta,
                                                      kernel_type, shp32)
        acc, last, med = _pixel_cutoff(acc, a32)
        np.testing.assert_array_equal(last, ncon[0, pid])
        np.testing.assert_array_equal(med, ncon[1, pid])
        median_j = med - 1
        if not acc.any():
            continue
        accT = torch.from_numpy(acc)
        u3 = torch.from_numpy(use3d)
        T = leaves["T"][ids]
        Tu, Tv, Tw = T[:, 0:3][None], T[:, 3:6][None], T[:, 6:9][None]
        pxd = torch.from_numpy(px.astype(np.float64))[:, None, None]
        pyd = torch.from_numpy(py.astype(np.float64))[:, None, None]
        k = pxd * Tw - Tu
        l = pyd * Tw - Tv
        p = torch.cross(k, l, dim=-1)
        p2 = torch.where(accT, p[..., 2], torch.ones_like(p[..., 2]))
        sx, sy = p[..., 0] / p2, p[..., 1] / p2
        rho3d = sx * sx + sy * sy
        xy = leaves["xy"][ids][None]
        dx = xy[..., 0] - pxd[..., 0]
        dy = xy[..., 1] - pyd[..., 0]
        rho2d = 2.0 * (dx * dx + dy * dy)
        rho = torch.where(u3, rho3d, rho2d)
        depth = torch.where(u3, (sx * Tw[..., 0] + sy * Tw[..., 1]) + Tw[..., 2], Tw[..., 2].expand_as(sx))
        rho_a = torch.where(accT, rho, torch.zeros_like(rho))
        if kernel_type != 0:
            G = _kernel_g(kernel_type, rho_a, leaves["shape"][ids][None].expand_as(rho_a), beta)
            G = torch.where(accT, G, torch.zeros_like(G))
        else:
            G = torch.exp(-0.5 * rho_a)
        if beta > 0 and kernel_type == 0:
            # the reference differentiates the position through -G' s with the
            # activated G' = (1+b) g / (1+b g) where the chain rule has -g s
            # (CR/backward.cu:1910-1913, :1977): value G', gradient scaled by G'/g
            Gp = (1.0 + beta) * G / (1.0 + beta * G)
            G = Gp.detach() + (Gp - Gp.detach()) * (Gp / G).detach()
        a_raw = leaves["opacity"][ids][None] * G
        alpha = a_raw - torch.relu(a_raw - 0.99).detach()
        alpha = torch.where(accT, alpha, torch.zeros_like(alpha))
        one_m = 1.0 - alpha
        Tcum = torch.cumprod(torch.cat([torch.ones_like(one_m[:, :1]), one_m[:, :-1]], dim=1), dim=1)
        w = alpha * Tcum
        # features
        if grid is None:
            feat = leaves["colors"][ids][None].expand(px.shape[0], n, C)
        else:
            rows = leaves.get("rows")
            if "hyb14" in grid:  # render mode 14: [rows | weight * grid | zeros], row ends with the weight
                # (the grid levels are skipped, value and gradient, when the weight is <= 1e-6)
                fs, nf = grid["hyb14"] * grid["F"], grid["L"] * grid["F"]
                hf = _hash_features(O, grid, leaves, ids, acc, use3d, sx32, sy32, sx, sy, homotrans_np, ap_level, nf)
                r = rows[ids][None].expand(px.shape[0], n, fs + 1)
                on = (r[..., fs:] > 1e-6).to(hf.dtype).detach()  # weights <= 1e-6 skip the grid
                feat = torch.cat([r[..., :fs], on * r[..., fs:] * hf,
                                  torch.zeros((px.shape[0], n, C - fs - nf), dtype=r.dtype)], dim=2)
            elif "hyb12" in grid:  # render mode 12: [coarse rows | blended levels | zeros], row ends with the weight
                fs, nf = grid["hyb12"] * grid["F"], grid["L"] * grid["F"]
                tdim = rows.shape[1] - 1
                hf = _hash_features(O, grid, leaves, ids, acc, use3d, sx32, sy32, sx, sy, homotrans_np, ap_level, nf)
                r = rows[ids][None].expand(px.shape[0], n, tdim + 1)
                wt = r[..., tdim:]
                nb = grid.get("nblend", nf)  # render mode 7 blends every channel, the grid zero past its levels
                hf = torch.cat([hf, torch.zeros_like(r[..., :nb - nf])], dim=2)
                feat = torch.cat([r[..., :fs], wt * r[..., fs:fs + nb] + (1.0 - wt) * hf,
                                  torch.zeros_like(r[..., :C - fs - nb])], dim=2)
            else:
                pgd = 0 if rows is None else rows.shape[1]
                feat = _hash_features(O, grid, leaves, ids, acc, use3d, sx32, sy32, sx, sy, homotrans_np, ap_level,
                                      C - pgd)
                if rows is not None:  # render mode 4: per-splat rows ahead of the grid features
                    feat = torch.cat([rows[ids][None].expand(px.shape[0], n, pgd), feat], dim=2)
        color[:, pid] = color[:, pid] + torch.einsum("pj,pjc->cp", w, feat)
        nrm = leaves["normal"][ids][None]
        m = FAR / (FAR - NEAR) * (1 - NEAR / torch.where(accT, depth, torch.ones_like(depth)))
        Aex = torch.cumsum(w, dim=1) - w
        M1ex = torch.cumsum(w * m, dim=1) - w * m
        M2ex = torch.cumsum(w * m * m, dim=1) - w * m * m
        dist = (w * (m * m * Aex + M2ex - 2 * m * M1ex)).sum(1)
        D = (w * torch.where(accT, depth, torch.zeros_like(depth))).sum(1)
        A = w.sum(1)
        N = torch.einsum("pj,pjc->cp", w, nrm.expand(px.shape[0], n, 3))
        mj = torch.from_numpy(np.clip(median_j, 0, n - 1))
        med = torch.gather(depth, 1, mj[:, None])[:, 0]
        med = torch.where(torch.from_numpy(median_j >= 0), med, torch.zeros_like(med))
        others[0, pid] = others[0, pid] + D
        others[1, pid] = others[1, pid] + A
        others[2:5, pid] = others[2:5, pid] + N
        others[5, pid] = others[5, pid] + med
        others[6, pid] = others[6, pid] + dist
    return color.reshape(C, H, W), others.reshape(7, H, W)


def _hash_features(O, grid, leaves, ids, acc, use3d, sx32, sy32, sx, sy, homo_np, ap_level, C):
    """Hash features [npix, n, C] of every pair (zero where not accepted),
    differentiable in homo (through xyz) and the table."""
    npix, n = acc.shape
    L, F, S, Hb = grid["L"], grid["F"], grid["S"], grid["H"]
    offsets = np.asarray(grid["offsets"], np.int64)
    vmin, vmax = grid["vmin"], grid["vmax"]
    Hm32 = homo_np[ids].reshape(1, n, 16)
    u3 = torch.from_numpy(use3d)
    xyz32 = np.where(use3d[..., None],
                     np.stack([sx32 * Hm32[..., 0] + sy32 * Hm32[..., 1] + Hm32[..., 3],
                               sx32 * Hm32[..., 4] + sy32 * Hm32[..., 5] + Hm32[..., 7],
                               sx32 * Hm32[..., 8] + sy32 * Hm32[..., 9] + Hm32[..., 11]], -1),
                     np.stack([Hm32[..., 3], Hm32[..., 7], Hm32[..., 11]], -1) + 0 * sx32[..., None])
    inv32 = f32(1.0) / (f32(vmax) - f32(vmin))
    with np.errstate(invalid="ignore"):
        u32 = (xyz32 - f32(vmin)) * inv32
        oob = ((u32 < 0) | (u32 > 1)).any(-1)
    hm = leaves["homo"][ids][None]
    xyz = torch.where(u3[..., None],
                      torch.stack([sx * hm[..., 0] + sy * hm[..., 1] + hm[..., 3],
                                   sx * hm[..., 4] + sy * hm[..., 5] + hm[..., 7],
                                   sx * hm[..., 8] + sy * hm[..., 9] + hm[..., 11]], -1),
                      torch.stack([hm[..., 3], hm[..., 7], hm[..., 11]], -1).expand(npix, n, 3))
    u = (xyz - vmin) / (vmax - vmin)
    apl = np.minimum(np.floor(ap_level[ids]).astype(np.int64), L)
    valid = acc & ~oob
    feat = torch.zeros((npix, n, C), dtype=torch.float64)
    table = leaves["table"]
    for lvl in range(L):
        scale, res = level_scale(O, S, Hb, lvl)
        hsize = int(offsets[lvl + 1] - offsets[lvl])
        x32 = u32 * scale + f32(0.5)
        with np.errstate(invalid="ignore"):
            g = np.where(valid[..., None], np.floor(x32), 0).astype(np.int64)
        pos = u * float(scale) + 0.5 - torch.from_numpy(g.astype(np.float64))
        use = valid & (lvl < apl)[None, :]
        usem = torch.from_numpy(use)
        acc_l = torch.zeros((npix, n, F), dtype=torch.float64)
        for corner in range(8):
            bits = [(corner >> d) & 1 for d in range(3)]
            wgt = torch.ones((npix, n), dtype=torch.float64)
            for d in range(3):
                wgt = wgt * (pos[..., d] if bits[d] else 1 - pos[..., d])
            q = g + np.array(bits, np.int64)
            idx = grid_index(False, hsize, res, q) + offsets[lvl]
            vals = table[torch.from_numpy(idx.reshape(-1))].reshape(npix, n, F)
            acc_l = acc_l + wgt[..., None] * vals
        feat[..., lvl * F:(lvl + 1) * F] = torch.where(usem[..., None], acc_l, torch.zeros_like(acc_l))
    return feat


def splat_forward(means, scales, rots, view, proj, W, H):
    """Per-splat transmat T [P,9] (scale modifier 1), screen centre with the
    cutoff-3 vector (9,9,-1) as the reference's backward differentiates it,
    view normal (normalised, facing the camera) and homotrans columns
    (R0 sx, R1 sy, p) of build_H.  rots are used unnormalised (the reference
    differentiates R(q) at the normalised q)."""
    w, x, y, z = rots[:, 0], rots[:, 1], rots[:, 2], rots[:, 3]
    R0 = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y + w * z), 2 * (x * z - w * y)], -1)
    R1 = torch.stack([2 * (x * y - w * z), 1 - 2 * (x * x + z * z), 2 * (y * z + w * x)], -1)
    R2 = torch.stack([2 * (x * z + w * y), 2 * (y * z - w * x), 1 - 2 * (x * x + y * y)], -1)
    L0 = R0 * scales[:, 0:1]
    L1 = R1 * scales[:, 1:2]
    A = torch.as_tensor(np.asarray(proj, np.float64).reshape(4, 4))       # A[r][c] = proj[4r+c]
    Np = torch.tensor([[W / 2.0, 0.0, 0.0, (W - 1) / 2.0], [0.0, H / 2.0, 0.0, (H - 1) / 2.0], [0.0, 0.0, 0.0, 1.0]],
                      dtype=torch.float64)                                # columns of ndc2pix
    Pm = A @ Np.T                                                         # [4,3]: P[r][c]
    ones = torch.ones_like(means[:, :1])
    zeros = torch.zeros_like(means[:, :1])
    Mrows = torch.stack([torch.cat([L0, zeros], -1), torch.cat([L1, zeros], -1), torch.cat([means, ones], -1)], 1)
    T = Mrows @ Pm                                                        # [P, 3(i), 3(c)]
    Tflat = T.transpose(1, 2).reshape(-1, 9)                              # [Tu(3) Tv(3) Tw(3)]
    Tu, Tv, Tw = T[:, :, 0], T[:, :, 1], T[:, :, 2]
    tv = torch.tensor([9.0, 9.0, -1.0], dtype=torch.float64)
    d = (tv * Tw * Tw).sum(-1, keepdim=True)
    f = tv / d
    xy = torch.stack([(f * Tu * Tw).sum(-1), (f * Tv * Tw).sum(-1)], -1)
    V = torch.as_tensor(np.asarray(view, np.float64).reshape(4, 4))       # V[r][c] = view[4r+c]
    n = R2 @ V[:3, :3]
    pv = means @ V[:3, :3] + V[3, :3]
    nn = n / n.norm(dim=-1, keepdim=True)
    sign = torch.where(-(pv * n).sum(-1) > 0, 1.0, -1.0).detach()
    nrm = nn * sign[:, None]
    homo = torch.stack([L0, L1, means], -1)                               # [P, 3(row), 3: col0, col1, col3]
    return Tflat, xy, nrm, homo
