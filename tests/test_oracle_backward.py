"""Pins the backward oracle (oracle/nest_oracle_bwd.c) against float64
automatic differentiation of an independent torch forward (tests/torch_ref.py)
on tiny scenes.  The torch forward is itself checked against the oracle's
forward outputs first, so the gradients are those of the forward the oracle
computes.  Tolerances are relative to each gradient array's largest entry:
the oracle runs in float32 and reconstructs T by division, the torch side is
float64 with exact products.  The largest error measured is 2.8e-5; the
1e-4 bound leaves 3.5x, while a dropped or mis-signed term is an O(1)
error.  The kernel types use 2e-4: the beta kernel's steeper position factor
raises the same entry's error (the splat's Tw.z, where the Gaussian gives
2.8e-5) to 9.0e-5, while the full derivative in place of the reference's
half factor is off by 0.47.
"""
import numpy as np
import pytest
import torch

import torch_ref as TR
from nest_splat.scene import get_spec, make_scene

TOL = 1e-4
TOL_KT = 2e-4


def _tiny(L=4, F=2, P=60, W=48, H=32, log_scale=-2.2, seed=0):
    spec = get_spec("cfg1", P=P, W=W, H=H, L=L, F=F, log2T=13, log_scale_mu=log_scale, name=f"tiny{seed}")
    sc = make_scene(spec)
    return sc


def _rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(np.abs(b).max(), 1e-30)
    return float(np.abs(a - b).max() / scale)


def _forward(oracle, sc, grid_on, beta=0.0, ap_level=None, kernel_type=0, shapes=None):
    sp = sc.spec
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    if grid_on:
        g = oracle.make_grid(sp.L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
        r = oracle.render(pre, b, W, H, sp.C, g, homotrans=sc.homotrans, ap_level=ap_level, beta=beta,
                          kernel_type=kernel_type, shapes=shapes)
    else:
        g = None
        colors = np.random.default_rng(5).uniform(0, 1, (sp.P, sp.C)).astype(np.float32)
        r = oracle.render(pre, b, W, H, sp.C, None, colors=colors, beta=beta, kernel_type=kernel_type, shapes=shapes)
        sc.__dict__["_colors"] = colors
    return pre, b, g, r, W, H


def kernel_shapes(kt, P, seed):
    """Per-splat kernel parameters in the ranges the reference trains them in:
    beta-kernel shapes 0.2-4, flex betas 0-2 (every 7th exactly 0, so that
    the splat falls back to the plain Gaussian), general exponents 2-8 (every
    9th below 2)."""
    rng = np.random.default_rng(seed)
    if kt == 1:
        return rng.uniform(0.2, 4.0, P).astype(np.float32)
    if kt == 2:
        v = rng.uniform(0.0, 2.0, P).astype(np.float32)
        v[::7] = 0.0
        return v
    v = rng.uniform(2.0, 8.0, P).astype(np.float32)
    v[::9] = rng.uniform(0.8, 2.0, v[::9].shape).astype(np.float32)
    return v


@pytest.mark.parametrize("grid_on,beta,kt", [(True, 0.0, 0), (False, 0.0, 0), (False, 1.5, 0), (True, 0.7, 0),
                                             (False, 0.0, 1), (True, 0.0, 1), (False, 0.0, 2), (False, 0.9, 2),
                                             (True, 0.0, 3), (False, 0.0, 3)])
def test_render_backward_matches_autograd(oracle, grid_on, beta, kt):
    """kernel_type 1-3 also pin dshapes, and their position terms follow the
    reference's factors (the beta kernel's is half the derivative, a flex
    splat without its own beta carries the settings' 1 + beta)."""
    sc = _tiny(seed=int(grid_on) * 2 + int(beta > 0) + 5 * kt)
    sp = sc.spec
    ap = sc.ap_level.reshape(-1).copy()
    ap[::3] = 2.0  # some splats query fewer levels
    shapes = None if kt == 0 else kernel_shapes(kt, sp.P, 40 + kt)
    pre, b, g, fwd, W, H = _forward(oracle, sc, grid_on, beta, ap, kt, shapes)
    assert b["num_rendered"] > 0
    rng = np.random.default_rng(11)
    dpix = rng.standard_normal(fwd["color"].shape).astype(np.float32)
    doth = rng.standard_normal(fwd["others"].shape).astype(np.float32)
    homo = sc.homotrans.reshape(-1, 16).astype(np.float32)
    gb = oracle.render_backward(pre, b, fwd, W, H, sp.C, g, dpix, doth, homotrans=homo if grid_on else None,
                                ap_level=ap, colors=None if grid_on else sc._colors, beta=beta, kernel_type=kt,
                                shapes=shapes)

    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    leaves = dict(T=leaf(pre["transmat"]), xy=leaf(pre["xy"]), normal=leaf(pre["normal_opacity"][:, :3]),
                  opacity=leaf(pre["normal_opacity"][:, 3]))
    if kt:
        leaves["shape"] = leaf(shapes)
    gd = None
    if grid_on:
        leaves["homo"] = leaf(homo)
        leaves["table"] = leaf(sc.table.reshape(-1, sp.F))
        gd = dict(L=sp.L, F=sp.F, S=sp.S, H=sp.base_res, offsets=sc.offsets, vmin=sp.gridrange[0],
                  vmax=sp.gridrange[1])
    else:
        leaves["colors"] = leaf(sc._colors)
    color, others = TR.render_forward(oracle, pre, b, fwd, W, H, sp.C, leaves, grid=gd, beta=beta,
                                      homotrans_np=homo, ap_level=ap, kernel_type=kt)
    # the torch forward is the oracle's forward
    assert _rel(color.detach().numpy(), fwd["color"]) < 1e-4
    assert _rel(others.detach().numpy(), fwd["others"][:7]) < 1e-3
    loss = (color * torch.from_numpy(dpix.astype(np.float64))).sum() + \
        (others * torch.from_numpy(doth[:7].astype(np.float64))).sum()
    loss.backward()

    vis = pre["radii"] > 0
    checks = {
        "dtransmat": (gb["dtransmat"], leaves["T"].grad),
        "dmean2D": (gb["dmean2D"][:, :2], leaves["xy"].grad),
        "dnormal": (gb["dnormal"], leaves["normal"].grad),
        "dopacity": (gb["dopacity"], leaves["opacity"].grad),
    }
    if grid_on:
        gh = leaves["homo"].grad.numpy()
        checks["dhomo"] = (gb["dhomo"], gh[:, [0, 4, 8, 1, 5, 9, 3, 7, 11]])
        checks["dtable"] = (gb["dtable"], leaves["table"].grad)
    else:
        checks["dcolors"] = (gb["dcolors"], leaves["colors"].grad)
    if kt:
        checks["dshapes"] = (gb["dshapes"], leaves["shape"].grad)
    for name, (ours, ref) in checks.items():
        ref = ref.numpy() if isinstance(ref, torch.Tensor) else ref
        if name != "dtable":
            ours, ref = ours[vis], ref[vis]
        assert np.abs(ref).max() > 0, name
        err = _rel(ours, ref)
        print(f"{name}: rel err {err:.2e}")
        assert err < (TOL_KT if kt else TOL), (name, err)


def test_preprocess_backward_matches_autograd(oracle):
    """compute_transmat_aabb backward: dL/dT, dL/dmean2D (through the
    reference's cutoff-3 centre), dL/dnormal and dL/dhomotrans to means,
    scales and rotations."""
    sc = _tiny(seed=7, P=40)
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    view, proj = cam.world_view_transform, cam.full_proj_transform
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, view, proj, W, H)
    vis = pre["radii"] > 0
    assert vis.sum() > 10
    P = sc.spec.P
    rng = np.random.default_rng(3)
    dT = rng.standard_normal((P, 9)).astype(np.float32)
    dxy = rng.standard_normal((P, 3)).astype(np.float32)
    dxy[:, 2] = 0
    dxy[::4, :2] = 0  # the fold is skipped when dL/dmean2D is zero
    dn = rng.standard_normal((P, 3)).astype(np.float32)
    dh = rng.standard_normal((P, 9)).astype(np.float32)
    gb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"], view, proj,
                                    W, H, dT, dh, dn, dxy)
    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    m, s, q = leaf(sc.means), leaf(sc.scales), leaf(sc.rotations)
    Tf, xy, nrm, homo = TR.splat_forward(m, s, q, view, proj, W, H)
    # the torch forward is the oracle's forward (T and the normal; scale modifier 1)
    assert _rel(Tf.detach().numpy()[vis], pre["transmat"][vis]) < 1e-5
    assert _rel(nrm.detach().numpy()[vis], pre["normal_opacity"][vis, :3]) < 1e-5
    t = lambda a: torch.from_numpy(np.asarray(a, np.float64))
    vm = t(vis.astype(np.float64))[:, None]
    loss = (t(dT) * Tf * vm).sum() + (t(dxy[:, :2]) * xy * vm).sum() + (t(dn) * nrm * vm).sum() + \
        (t(dh).reshape(P, 3, 3).transpose(1, 2) * homo * vm[:, :, None]).sum()
    loss.backward()
    for name, ref in (("dmeans", m.grad), ("dscales", s.grad), ("drots", q.grad)):
        err = _rel(gb[name][vis], ref.numpy()[vis])
        print(f"{name}: rel err {err:.2e}")
        assert err < TOL, (name, err)
    # splats culled by preprocess get nothing
    assert not gb["dmeans"][~vis].any() and not gb["drots"][~vis].any()


def _sh_forward_torch(means, shs, campos, deg):
    """computeColorFromSH (CR/forward.cu:21-72) in float64 torch."""
    C0, C1 = 0.28209479177387814, 0.4886025119029199
    C2 = [1.0925484305920792, -1.0925484305920792, 0.31539156525252005, -1.0925484305920792, 0.5462742152960396]
    C3 = [-0.5900435899266435, 2.890611442640554, -0.4570457994644658, 0.3731763325901154, -0.4570457994644658,
          1.445305721320277, -0.5900435899266435]
    d = means - torch.as_tensor(np.asarray(campos, np.float64))
    d = d / d.norm(dim=-1, keepdim=True)
    x, y, z = d[:, 0:1], d[:, 1:2], d[:, 2:3]
    sh = lambda i: shs[:, i, :]
    r = C0 * sh(0)
    if deg > 0:
        r = r - C1 * y * sh(1) + C1 * z * sh(2) - C1 * x * sh(3)
    if deg > 1:
        xx, yy, zz, xy, yz, xz = x * x, y * y, z * z, x * y, y * z, x * z
        r = r + C2[0] * xy * sh(4) + C2[1] * yz * sh(5) + C2[2] * (2 * zz - xx - yy) * sh(6) + \
            C2[3] * xz * sh(7) + C2[4] * (xx - yy) * sh(8)
    if deg > 2:
        r = r + C3[0] * y * (3 * xx - yy) * sh(9) + C3[1] * xy * z * sh(10) + C3[2] * y * (4 * zz - xx - yy) * sh(11) + \
            C3[3] * z * (2 * zz - 3 * xx - 3 * yy) * sh(12) + C3[4] * x * (4 * zz - xx - yy) * sh(13) + \
            C3[5] * z * (xx - yy) * sh(14) + C3[6] * x * (xx - 3 * yy) * sh(15)
    r = r + 0.5
    return torch.clamp_min(r, 0.0)


@pytest.mark.parametrize("deg", [0, 1, 2, 3])
def test_sh_backward_matches_autograd(oracle, deg):
    sc = _tiny(seed=9, P=40)
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    view, proj = cam.world_view_transform, cam.full_proj_transform
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, view, proj, W, H)
    vis = pre["radii"] > 0
    P = sc.spec.P
    rng = np.random.default_rng(deg)
    shs = (rng.standard_normal((P, 16, 3)) * 2.0).astype(np.float32)
    campos = np.asarray(cam.camera_center, np.float32)
    rgb, clamped = oracle.sh_colors(pre, sc.means, campos, shs, deg)
    assert clamped.any() and not clamped.all()
    dcol = rng.standard_normal((P, 3)).astype(np.float32)
    z = np.zeros((P, 9), np.float32)
    gb = oracle.preprocess_backward(sc.means, sc.scales, sc.rotations, pre["radii"], pre["transmat"], view, proj,
                                    W, H, z, z, np.zeros((P, 3), np.float32), np.zeros((P, 3), np.float32),
                                    shs=shs, sh_degree=deg, campos=campos, clamped=clamped, dcolors=dcol)
    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    m, sh = leaf(sc.means), leaf(shs)
    col = _sh_forward_torch(m, sh, campos, deg)
    assert _rel(col.detach().numpy()[vis], rgb[vis]) < 1e-5
    (col * torch.from_numpy(dcol.astype(np.float64)) * torch.from_numpy(vis.astype(np.float64))[:, None]).sum().backward()
    nco = (deg + 1) ** 2
    err_sh = _rel(gb["dshs"][vis][:, :nco], sh.grad.numpy()[vis][:, :nco])
    err_m = _rel(gb["dmeans"][vis], m.grad.numpy()[vis]) if deg > 0 else 0.0
    print(f"deg {deg}: dshs {err_sh:.2e} dmeans {err_m:.2e}")
    assert err_sh < TOL and err_m < TOL
    assert not gb["dshs"][:, nco:].any()


@pytest.mark.parametrize("interp,align", [(0, False), (1, False), (0, True)])
def test_grid_encode_backward_matches_autograd(oracle, interp, align):
    """kernel_grid_backward + kernel_input_backward with the forward's dy_dx
    (GE/src/gridencoder.cu:196-366), including out-of-range inputs."""
    L, F, S, Hb = 5, 2, float(np.log2(1.6)), 8
    rng = np.random.default_rng(interp * 2 + int(align))
    sizes = [min(2 ** 12, -(-((int(np.ceil(np.exp2(l * S) * Hb - 1)) + 1 + (0 if align else 1)) ** 3) // 8) * 8)
             for l in range(L)]
    offsets = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    table = (rng.standard_normal((int(offsets[-1]), F)) * 0.3).astype(np.float32)
    B = 300
    x = rng.uniform(-0.05, 1.05, (B, 3)).astype(np.float32)
    grid = oracle.make_grid(L, F, S, Hb, offsets, table, (0.0, 1.0), False, align_corners=align, interp=interp)
    out = oracle.grid_encode(grid, x)
    g = rng.standard_normal(out.shape).astype(np.float32)
    gt, gi = oracle.grid_encode_backward(grid, x, g)
    # autograd of the same interpolation in float64
    xt = torch.tensor(x.astype(np.float64), requires_grad=True)
    tt = torch.tensor(table.astype(np.float64), requires_grad=True)
    oob = ((x < 0) | (x > 1)).any(1)
    res = torch.zeros((B, L * F), dtype=torch.float64)
    for l in range(L):
        scale, rs = TR.level_scale(oracle, S, Hb, l)
        hsize = int(offsets[l + 1] - offsets[l])
        x32 = x * scale + np.float32(0.0 if align else 0.5)
        gg = np.floor(x32).astype(np.int64)
        pos = xt * float(scale) + (0.0 if align else 0.5) - torch.from_numpy(gg.astype(np.float64))
        if interp == 1:
            pos = pos * pos * (3 - 2 * pos)
        acc = torch.zeros((B, F), dtype=torch.float64)
        for corner in range(8):
            bits = [(corner >> d) & 1 for d in range(3)]
            wgt = torch.ones(B, dtype=torch.float64)
            for d in range(3):
                wgt = wgt * (pos[:, d] if bits[d] else 1 - pos[:, d])
            idx = TR.grid_index(align, hsize, rs, np.clip(gg, 0, None) + np.array(bits)) + offsets[l]
            acc = acc + wgt[:, None] * tt[torch.from_numpy(idx)]
        res[:, l * F:(l + 1) * F] = torch.where(torch.from_numpy(oob)[:, None], torch.zeros_like(acc), acc)
    assert _rel(res.detach().numpy(), out) < 1e-5
    (res * torch.from_numpy(g.astype(np.float64))).sum().backward()
    e_t, e_i = _rel(gt, tt.grad.numpy()), _rel(gi, xt.grad.numpy())
    print(f"interp {interp} align {align}: grad_table {e_t:.2e} grad_inputs {e_i:.2e}")
    assert e_t < TOL and e_i < TOL
    assert not gi[oob].any()


@pytest.mark.parametrize("hyb,active", [(2, 4), (1, 2), (3, 0)])
def test_cat_mode_backward_matches_autograd(oracle, hyb, active):
    """Render mode 4 backward (CR/backward.cu:987-1040): per-splat rows ahead
    of the grid features.  With every grid level active it is the gradient of
    the forward.  With fewer active levels the reference differentiates only
    the active ones and takes the features past them as zero when it rebuilds
    the blend (the offsets are copied only up to the active count,
    CR/backward.cu:576-612), so its gradients are those of the forward over a
    grid of the active levels alone, though the forward rendered them all."""
    sc = _tiny(seed=20 + hyb)
    sp = sc.spec
    F, L = sp.F, sp.L
    pgd = hyb * F
    C = pgd + L * F + 2
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    ap = sc.ap_level.reshape(-1).copy()
    ap[::3] = 2.0
    rows = np.random.default_rng(hyb).uniform(-1, 1, (sp.P, pgd)).astype(np.float32)
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    assert b["num_rendered"] > 0
    g = oracle.make_grid(L, sp.F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    level = ((hyb + L) << 16) | (active << 8) | hyb
    fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=4,
                        level=level)
    rng = np.random.default_rng(13)
    dpix = rng.standard_normal(fwd["color"].shape).astype(np.float32)
    doth = rng.standard_normal(fwd["others"].shape).astype(np.float32)
    homo = sc.homotrans.reshape(-1, 16).astype(np.float32)
    gb = oracle.render_backward(pre, b, fwd, W, H, C, g, dpix, doth, homotrans=homo, ap_level=ap, colors=rows,
                                render_mode=4, level=level)
    assert gb["dcolors"].shape == (sp.P, pgd)

    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    leaves = dict(T=leaf(pre["transmat"]), xy=leaf(pre["xy"]), normal=leaf(pre["normal_opacity"][:, :3]),
                  opacity=leaf(pre["normal_opacity"][:, 3]), homo=leaf(homo),
                  table=leaf(sc.table.reshape(-1, sp.F)), rows=leaf(rows))
    gd = dict(L=min(active, L), F=F, S=sp.S, H=sp.base_res, offsets=sc.offsets, vmin=sp.gridrange[0],
              vmax=sp.gridrange[1])
    color, others = TR.render_forward(oracle, pre, b, fwd, W, H, C, leaves, grid=gd, homotrans_np=homo,
                                      ap_level=ap)
    nf = pgd + min(active, L) * F
    assert _rel(color.detach().numpy()[:nf], fwd["color"][:nf]) < 1e-4
    if active < L:
        assert np.abs(fwd["color"][nf:pgd + L * F]).max() > 0  # rendered, not differentiated
    loss = (color * torch.from_numpy(dpix.astype(np.float64))).sum() + \
        (others * torch.from_numpy(doth[:7].astype(np.float64))).sum()
    loss.backward()
    vis = pre["radii"] > 0
    checks = {"dtransmat": (gb["dtransmat"], leaves["T"].grad), "dmean2D": (gb["dmean2D"][:, :2], leaves["xy"].grad),
              "dnormal": (gb["dnormal"], leaves["normal"].grad), "dopacity": (gb["dopacity"], leaves["opacity"].grad),
              "dcolors": (gb["dcolors"], leaves["rows"].grad)}
    if active > 0:
        gh = leaves["homo"].grad.numpy()
        checks["dhomo"] = (gb["dhomo"], gh[:, [0, 4, 8, 1, 5, 9, 3, 7, 11]])
        checks["dtable"] = (gb["dtable"], leaves["table"].grad)
    else:
        assert not gb["dtable"].any() and not gb["dhomo"].any()
    for name, (ours, ref) in checks.items():
        ref = ref.numpy() if isinstance(ref, torch.Tensor) else ref
        if name != "dtable":
            ours, ref = ours[vis], ref[vis]
        assert np.abs(ref).max() > 0, name
        err = _rel(ours, ref)
        print(f"{name}: rel err {err:.2e}")
        assert err < TOL, (name, err)
    if 0 < active < L:  # no gradient reaches the inactive levels
        assert not gb["dtable"][int(sc.offsets[active]):].any()


@pytest.mark.parametrize("hyb,hl,extra,ap_cap", [(2, 3, 1, False), (1, 4, 0, True), (3, 0, 1, False)])
def test_adaptive_cat_backward_matches_autograd(oracle, hyb, hl, extra, ap_cap):
    """Render mode 12 training backward (CR/backward.cu:1425-1520): coarse rows
    unweighted, the hl grid levels blended with the row by its weight; the
    gradients of the rows (weight included), the table and the geometry are
    those of the forward.  Per-splat weights in (0, 1); some splats query
    fewer levels (ap_level 2)."""
    sc = _tiny(seed=30 + hyb)
    sp = sc.spec
    F = sp.F
    total = hyb + hl + extra
    tdim, fs = total * F, hyb * F
    C = tdim
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    ap = sc.ap_level.reshape(-1).copy()
    if ap_cap:
        ap[::3] = 2.0
    rng = np.random.default_rng(hyb + hl)
    rows = rng.uniform(-1, 1, (sp.P, tdim + 1)).astype(np.float32)
    rows[:, tdim] = rng.uniform(0.05, 0.95, sp.P).astype(np.float32)
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    assert b["num_rendered"] > 0
    g = oracle.make_grid(max(hl, 1), F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    level = (total << 16) | (hl << 8) | hyb
    fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=12,
                        level=level)
    r2 = np.random.default_rng(17)
    dpix = r2.standard_normal(fwd["color"].shape).astype(np.float32)
    doth = r2.standard_normal(fwd["others"].shape).astype(np.float32)
    homo = sc.homotrans.reshape(-1, 16).astype(np.float32)
    gb = oracle.render_backward(pre, b, fwd, W, H, C, g, dpix, doth, homotrans=homo, ap_level=ap, colors=rows,
                                render_mode=12, level=level)
    assert gb["dcolors"].shape == (sp.P, tdim + 1)

    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    leaves = dict(T=leaf(pre["transmat"]), xy=leaf(pre["xy"]), normal=leaf(pre["normal_opacity"][:, :3]),
                  opacity=leaf(pre["normal_opacity"][:, 3]), homo=leaf(homo),
                  table=leaf(sc.table.reshape(-1, sp.F)), rows=leaf(rows))
    gd = dict(L=hl, F=F, S=sp.S, H=sp.base_res, offsets=sc.offsets, vmin=sp.gridrange[0], vmax=sp.gridrange[1],
              hyb12=hyb)
    color, others = TR.render_forward(oracle, pre, b, fwd, W, H, C, leaves, grid=gd, homotrans_np=homo,
                                      ap_level=ap)
    assert _rel(color.detach().numpy(), fwd["color"]) < 1e-4
    loss = (color * torch.from_numpy(dpix.astype(np.float64))).sum() + \
        (others * torch.from_numpy(doth[:7].astype(np.float64))).sum()
    loss.backward()
    vis = pre["radii"] > 0
    rg = leaves["rows"].grad.numpy()
    checks = {"dtransmat": (gb["dtransmat"], leaves["T"].grad), "dmean2D": (gb["dmean2D"][:, :2], leaves["xy"].grad),
              "dnormal": (gb["dnormal"], leaves["normal"].grad), "dopacity": (gb["dopacity"], leaves["opacity"].grad),
              "drows": (gb["dcolors"][:, :tdim], rg[:, :tdim])}
    if hl > 0:
        gh = leaves["homo"].grad.numpy()
        checks["dhomo"] = (gb["dhomo"], gh[:, [0, 4, 8, 1, 5, 9, 3, 7, 11]])
        checks["dtable"] = (gb["dtable"], leaves["table"].grad)
        checks["dweight"] = (gb["dcolors"][:, tdim], rg[:, tdim])
    else:
        assert not gb["dtable"].any() and not gb["dcolors"][:, tdim].any()
    for name, (ours, ref) in checks.items():
        ref = ref.numpy() if isinstance(ref, torch.Tensor) else ref
        if name != "dtable":
            ours, ref = ours[vis], ref[vis]
        assert np.abs(ref).max() > 0, name
        err = _rel(ours, ref)
        print(f"{name}: rel err {err:.2e}")
        assert err < TOL, (name, err)


@pytest.mark.parametrize("hyb,hl,ap_cap", [(2, 3, True), (1, 4, False), (3, 0, False)])
def test_adaptive_zero_backward_matches_autograd(oracle, hyb, hl, ap_cap):
    """Render mode 14 training backward (CR/backward.cu:1521-1590): coarse rows,
    then the grid levels times the row's weight; the gradients of the rows
    (weight included), the table and the geometry are those of the forward.
    A few splats carry weight 0 (their grid levels are skipped)."""
    sc = _tiny(seed=40 + hyb)
    sp = sc.spec
    F = sp.F
    total = hyb + hl + 1
    pgd, C = hyb * F, total * F
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    ap = sc.ap_level.reshape(-1).copy()
    if ap_cap:
        ap[::3] = 2.0
    rng = np.random.default_rng(hyb + hl + 5)
    rows = rng.uniform(-1, 1, (sp.P, pgd + 1)).astype(np.float32)
    rows[:, pgd] = rng.uniform(0.05, 0.95, sp.P).astype(np.float32)
    rows[::7, pgd] = 0.0
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(max(hl, 1), F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    level = (total << 16) | (hl << 8) | hyb
    fwd = oracle.render(pre, b, W, H, C, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=14,
                        level=level)
    r2 = np.random.default_rng(19)
    dpix = r2.standard_normal(fwd["color"].shape).astype(np.float32)
    doth = r2.standard_normal(fwd["others"].shape).astype(np.float32)
    homo = sc.homotrans.reshape(-1, 16).astype(np.float32)
    gb = oracle.render_backward(pre, b, fwd, W, H, C, g, dpix, doth, homotrans=homo, ap_level=ap, colors=rows,
                                render_mode=14, level=level)
    assert gb["dcolors"].shape == (sp.P, pgd + 1)
    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    leaves = dict(T=leaf(pre["transmat"]), xy=leaf(pre["xy"]), normal=leaf(pre["normal_opacity"][:, :3]),
                  opacity=leaf(pre["normal_opacity"][:, 3]), homo=leaf(homo),
                  table=leaf(sc.table.reshape(-1, sp.F)), rows=leaf(rows))
    gd = dict(L=hl, F=F, S=sp.S, H=sp.base_res, offsets=sc.offsets, vmin=sp.gridrange[0], vmax=sp.gridrange[1],
              hyb14=hyb)
    color, others = TR.render_forward(oracle, pre, b, fwd, W, H, C, leaves, grid=gd, homotrans_np=homo,
                                      ap_level=ap)
    assert _rel(color.detach().numpy(), fwd["color"]) < 1e-4
    loss = (color * torch.from_numpy(dpix.astype(np.float64))).sum() + \
        (others * torch.from_numpy(doth[:7].astype(np.float64))).sum()
    loss.backward()
    vis = pre["radii"] > 0
    rg = leaves["rows"].grad.numpy()
    checks = {"dtransmat": (gb["dtransmat"], leaves["T"].grad), "dmean2D": (gb["dmean2D"][:, :2], leaves["xy"].grad),
              "dnormal": (gb["dnormal"], leaves["normal"].grad), "dopacity": (gb["dopacity"], leaves["opacity"].grad),
              "drows": (gb["dcolors"][:, :pgd], rg[:, :pgd])}
    if hl > 0:
        gh = leaves["homo"].grad.numpy()
        checks["dhomo"] = (gb["dhomo"], gh[:, [0, 4, 8, 1, 5, 9, 3, 7, 11]])
        checks["dtable"] = (gb["dtable"], leaves["table"].grad)
        checks["dweight"] = (gb["dcolors"][:, pgd], rg[:, pgd])
    for name, (ours, ref) in checks.items():
        ref = ref.numpy() if isinstance(ref, torch.Tensor) else ref
        if name != "dtable":
            ours, ref = ours[vis], ref[vis]
        assert np.abs(ref).max() > 0, name
        err = _rel(ours, ref)
        print(f"{name}: rel err {err:.2e}")
        assert err < TOL, (name, err)


@pytest.mark.parametrize("hl,extra,ap_cap", [(3, 2, True), (4, 0, False)])
def test_adaptive_add_backward_matches_autograd(oracle, hl, extra, ap_cap):
    """Render mode 7 backward (CR/backward.cu:1108-1189): weight * row +
    (1 - weight) * grid over all total*F channels.  The rows' and the grid's
    gradients are the forward's; the weight slot holds the gradient times
    weight * (1 - weight), the reference's gradient of the logit whose
    sigmoid the weight is."""
    sc = _tiny(seed=50 + hl)
    sp = sc.spec
    F = sp.F
    total = hl + extra
    tdim = total * F
    cam = sc.cameras[0]
    W, H = cam.image_width, cam.image_height
    ap = sc.ap_level.reshape(-1).copy()
    if ap_cap:
        ap[::3] = 2.0
    rng = np.random.default_rng(hl + 70)
    rows = rng.uniform(-1, 1, (sp.P, tdim + 1)).astype(np.float32)
    rows[:, tdim] = rng.uniform(0.05, 0.95, sp.P).astype(np.float32)
    pre = oracle.preprocess(sc.means, sc.scales, sc.rotations, sc.opacity, cam.world_view_transform,
                            cam.full_proj_transform, W, H)
    b = oracle.binning(pre, W, H)
    g = oracle.make_grid(hl, F, sp.S, sp.base_res, sc.offsets, sc.table, sp.gridrange, sp.contract)
    level = (total << 16) | (hl << 8)
    fwd = oracle.render(pre, b, W, H, tdim, g, homotrans=sc.homotrans, ap_level=ap, colors=rows, render_mode=7,
                        level=level)
    r2 = np.random.default_rng(23)
    dpix = r2.standard_normal(fwd["color"].shape).astype(np.float32)
    doth = r2.standard_normal(fwd["others"].shape).astype(np.float32)
    homo = sc.homotrans.reshape(-1, 16).astype(np.float32)
    gb = oracle.render_backward(pre, b, fwd, W, H, tdim, g, dpix, doth, homotrans=homo, ap_level=ap, colors=rows,
                                render_mode=7, level=level)
    leaf = lambda a: torch.tensor(np.asarray(a, np.float64), requires_grad=True)
    leaves = dict(T=leaf(pre["transmat"]), xy=leaf(pre["xy"]), normal=leaf(pre["normal_opacity"][:, :3]),
                  opacity=leaf(pre["normal_opacity"][:, 3]), homo=leaf(homo),
                  table=leaf(sc.table.reshape(-1, sp.F)), rows=leaf(rows))
    gd = dict(L=hl, F=F, S=sp.S, H=sp.base_res, offsets=sc.offsets, vmin=sp.gridrange[0], vmax=sp.gridrange[1],
              hyb12=0, nblend=tdim)
    color, others = TR.render_forward(oracle, pre, b, fwd, W, H, tdim, leaves, grid=gd, homotrans_np=homo,
                                      ap_level=ap)
    assert _rel(color.detach().numpy(), fwd["color"]) < 1e-4
    loss = (color * torch.from_numpy(dpix.astype(np.float64))).sum() + \
        (others * torch.from_numpy(doth[:7].astype(np.float64))).sum()
    loss.backward()
    vis = pre["radii"] > 0
    rg = leaves["rows"].grad.numpy()
    w = rows[:, tdim].astype(np.float64)
    gh = leaves["homo"].grad.numpy()
    checks = {"dtransmat": (gb["dtransmat"], leaves["T"].grad), "dopacity": (gb["dopacity"], leaves["opacity"].grad),
              "drows": (gb["dcolors"][:, :tdim], rg[:, :tdim]), "dtable": (gb["dtable"], leaves["table"].grad),
              "dhomo": (gb["dhomo"], gh[:, [0, 4, 8, 1, 5, 9, 3, 7, 11]]),
              "dlogit": (gb["dcolors"][:, tdim], rg[:, tdim] * w * (1.0 - w))}
    for name, (ours, ref) in checks.items():
        ref = ref.numpy() if isinstance(ref, torch.Tensor) else ref
        if name != "dtable":
            ours, ref = ours[vis], ref[vis]
        assert np.abs(ref).max() > 0, name
        err = _rel(ours, ref)
        print(f"{name}: rel err {err:.2e}")
        assert err < TOL, (name, err)
