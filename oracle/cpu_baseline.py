"""CPU baseline of the forward path in the form the benchmark names: a NumPy
transcription of renderCUDAsurfelForward's per-pixel loop (mode 0),
vectorised over the 256 pixels of a tile and parallel over tiles with a
process pool, plus torch-CPU hash encode of the accepted hits, torch-CPU MLP
decode and torch-CPU RVQ gather-sum.

TEST INFRASTRUCTURE ONLY: run by bench.py's cpu_baseline leg (as a child
process, `python -m oracle.cpu_baseline`) and by tests/, never by the product
package.  It is a timed baseline, not the parity oracle: its float sums run
in a different order (features are added per hit after the loop, NumPy and
torch pick their own exp), so it agrees with oracle/nest_oracle.c to ~1e-5
relative, not bit for bit (tests/test_cpu_baseline.py).

Reference semantics followed (paths relative to the reference root):
- per-pixel loop: submodules/diff-surfel-rasterization/cuda_rasterizer/
  forward.cu:834-971 (intersection, rho, alpha, early stop), :1127-1145
  (mode-0 hash lookup at the 3D hit), :1914-1916 (feature accumulation),
  :1945-1957 (appearance colour), :2008-2048 (outputs);
- hash encode: cuda_rasterizer/hashgrid.h:7-212 (contract, per-level scale,
  dense/hashed index, trilinear weights);
- MLP: hash_encoder/modules.py:587-602 (SH16 of (d+1)/2, ReLU, ReLU, sigmoid,
  no biases); RVQ: the benchmark's ordered stage sum.
Preprocess and binning come from the C oracle (single thread) and are timed
with it.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for _p in (os.path.join(ROOT, "nest-splatting_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

NEAR, FAR = np.float32(0.2), np.float32(100.0)
BLOCK = 16

# Scene arrays shared with the forked pool workers (set before the pool starts).
_STATE: dict = {}


def render_tile(tile: int):
    """One tile, mode 0 with a hash grid: returns (pixel ids [n], allmap rows
    [14, 256] minus the features, final T [256], and the accepted hits as
    (local pixel, xyz [3], weight, ap) arrays in hit order)."""
    S = _STATE
    W, H, gx = S["W"], S["H"], S["gx"]
    tx, ty = tile % gx, tile // gx
    lx, ly = np.meshgrid(np.arange(BLOCK), np.arange(BLOCK), indexing="xy")
    px = (tx * BLOCK + lx).reshape(-1)
    py = (ty * BLOCK + ly).reshape(-1)
    inside = (px < W) & (py < H)
    pxf, pyf = px.astype(np.float32), py.astype(np.float32)
    n = BLOCK * BLOCK
    T = np.ones(n, np.float32)
    done = ~inside
    contributor = np.zeros(n, np.uint32)
    render_number = np.zeros(n, np.float32)
    D = np.zeros(n, np.float32)
    M1 = np.zeros(n, np.float32)
    M2 = np.zeros(n, np.float32)
    dist = np.zeros(n, np.float32)
    med = np.zeros(n, np.float32)
    Nrm = np.zeros((3, n), np.float32)
    pos = np.zeros((3, n), np.float32)
    vis = np.zeros((2, n), np.float32)
    mfac = np.float32(FAR / (FAR - NEAR))
    hit_pix, hit_xyz, hit_w, hit_ap = [], [], [], []
    r0, r1 = S["ranges"][tile]
    tm, xy, no, hm, apl = S["transmat"], S["xy"], S["normal_opacity"], S["homotrans"], S["ap"]
    for e in range(int(r0), int(r1)):
        if done.all():
            break
        i = int(S["point_list"][e])
        act = ~done
        contributor += act
        Tu, Tv, Tw = tm[i, 0:3], tm[i, 3:6], tm[i, 6:9]
        k0, k1, k2 = pxf * Tw[0] - Tu[0], pxf * Tw[1] - Tu[1], pxf * Tw[2] - Tu[2]
        l0, l1, l2 = pyf * Tw[0] - Tv[0], pyf * Tw[1] - Tv[1], pyf * Tw[2] - Tv[2]
        p0, p1, p2 = k1 * l2 - k2 * l1, k2 * l0 - k0 * l2, k0 * l1 - k1 * l0
        with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
            sx, sy = p0 / p2, p1 / p2
            rho3d = sx * sx + sy * sy
            dx, dy = xy[i, 0] - pxf, xy[i, 1] - pyf
            rho2d = np.float32(2.0) * (dx * dx + dy * dy)
            use3d = rho3d <= rho2d
            rho = np.minimum(rho3d, rho2d)
            depth = np.where(use3d, (sx * Tw[0] + sy * Tw[1]) + Tw[2], Tw[2]).astype(np.float32)
            power = np.float32(-0.5) * rho
            G = np.exp(power)
            alpha = np.minimum(np.float32(0.99), no[i, 3] * G)
        ok = act & (p2 != 0) & (depth >= NEAR) & (power <= 0) & (alpha >= np.float32(1.0 / 255.0))
        test_T = T * (np.float32(1) - alpha)
        stop = ok & (test_T < np.float32(1e-4))
        done |= stop
        ok &= ~stop
        if not ok.any():
            continue
        w = np.where(ok, alpha * T, np.float32(0))
        render_number += ok
        m = mfac * (np.float32(1) - NEAR / depth)
        Aa = np.float32(1) - T
        dist = np.where(ok, dist + (m * m * Aa + M2 - np.float32(2) * m * M1) * w, dist)
        D += np.where(ok, depth * w, 0)
        M1 += np.where(ok, m * w, 0)
        M2 += np.where(ok, m * m * w, 0)
        med = np.where(ok & (T > np.float32(0.5)), depth, med)
        Nrm += np.where(ok, no[i, :3, None] * w, 0)
        Hm = hm[i]
        xyz = np.where(use3d, np.stack([sx * Hm[0] + sy * Hm[1] + Hm[3], sx * Hm[4] + sy * Hm[5] + Hm[7],
                                        sx * Hm[8] + sy * Hm[9] + Hm[11]]), Hm[[3, 7, 11], None])
        pos += np.where(ok, w * xyz, 0)
        ap = int(apl[i])
        apc = (np.float32((ap - 2) * 0.5), np.float32(1.0)) if ap <= 4 else (np.float32(1.0), np.float32(1.0 - (ap - 4) * 0.5))
        vis[0] += np.where(ok, apc[0] * w, 0)
        vis[1] += np.where(ok, apc[1] * w, 0)
        idx = np.nonzero(ok)[0]
        hit_pix.append(idx)
        hit_xyz.append(xyz[:, idx].T)
        hit_w.append(w[idx])
        hit_ap.append(np.full(idx.size, ap, np.int32))
        T = np.where(ok, test_T, T)
    others = np.stack([D, 1 - T, Nrm[0], Nrm[1], Nrm[2], med, dist, render_number, pos[0], pos[1], pos[2], vis[0],
                       vis[1], np.zeros(n, np.float32)])
    pix = (py * W + px)
    cat = (lambda a, shape, dt: np.concatenate(a) if a else np.zeros(shape, dt))
    return (pix[inside], others[:, inside], cat(hit_pix, (0,), np.int64), cat(hit_xyz, (0, 3), np.float32),
            cat(hit_w, (0,), np.float32), cat(hit_ap, (0,), np.int32), inside)


def hash_encode_torch(xyz, ap, grid: dict):
    """query_feature of N points (hashgrid.h:53-212) in torch on the CPU:
    [N, L*F] features, zero past min(ap, L) levels and for points out of the
    grid (non-contract mode)."""
    import torch
    L, F, S, Hb = grid["L"], grid["F"], grid["S"], grid["H"]
    table = grid["table_t"]
    offs = grid["offsets"]
    x = torch.from_numpy(xyz)
    vmin, vmax = grid["range"]
    f32 = np.float32
    if grid["contract"]:
        vmid = float(f32(f32(vmax + vmin) * f32(0.5)))
        inv = float(f32(1) / f32(f32(vmax - vmin) * f32(0.5)))
        u = (x - vmid) * inv
        nrm = torch.sqrt((u[:, 0:1] * u[:, 0:1] + u[:, 1:2] * u[:, 1:2]) + u[:, 2:3] * u[:, 2:3])
        inv_n = 1 / nrm
        st = torch.where(nrm <= 1, torch.ones_like(nrm), (2 - inv_n) * inv_n)
        u = (st * u + 2) * 0.25
        oob = torch.zeros(u.shape[0], dtype=torch.bool)
    else:
        u = (x - vmin) * float(f32(1) / f32(vmax - vmin))
        oob = ((u < 0) | (u > 1)).any(dim=1)
    apt = torch.from_numpy(ap)
    out = torch.zeros((u.shape[0], L * F), dtype=torch.float32)
    for l in range(L):
        # scale = 2^(l S) H - 1 and resolution ceil(scale) + 1 in float32
        # (hashgrid.h:122-124); the dense stride is resolution + 1
        # (get_grid_index, hashgrid.h:7-40), dense while stride^3 fits the level
        scale = np.float32(np.exp2(np.float64(np.float32(l) * np.float32(S)))) * np.float32(Hb) - np.float32(1)
        stride = int(np.ceil(scale)) + 2
        hsize = int(offs[l + 1] - offs[l])
        dense = stride ** 3 <= hsize
        posf = u * float(scale) + 0.5
        g = torch.floor(posf).clamp(min=0).to(torch.int64)
        fr = posf - g.to(torch.float32)
        acc = torch.zeros((u.shape[0], F), dtype=torch.float32)
        for c in range(8):
            b = [(c >> d) & 1 for d in range(3)]
            wgt = torch.ones(u.shape[0], dtype=torch.float32)
            for d in range(3):
                wgt = wgt * (fr[:, d] if b[d] else 1 - fr[:, d])
            q = g + torch.tensor(b, dtype=torch.int64)
            if dense:
                idx = q[:, 0] + q[:, 1] * stride + q[:, 2] * stride * stride
            else:
                idx = (q[:, 0] ^ ((q[:, 1] * 2654435761) & 0xFFFFFFFF) ^ ((q[:, 2] * 805459861) & 0xFFFFFFFF))
            idx = (idx & 0xFFFFFFFF) % hsize + int(offs[l])
            acc += wgt[:, None] * table[idx]
        keep = (~oob) & (apt > l)
        out[:, l * F:(l + 1) * F] = torch.where(keep[:, None], acc, torch.zeros_like(acc))
    return out


def mlp_torch(feat, dirs, W1, W2, W3):
    """rgb_decode (hash_encoder/modules.py:587-602) in fp32 torch on the CPU:
    [N, C] features and [N, 3] unit directions to [N, 3]."""
    import torch
    u = (torch.from_numpy(dirs) + 1) / 2
    x, y, z = (2 * u - 1).unbind(1)
    xy, xz, yz, x2, y2, z2 = x * y, x * z, y * z, x * x, y * y, z * z
    sh = torch.stack([torch.full_like(x, 0.28209479177387814), -0.48860251190291987 * y, 0.48860251190291987 * z,
                      -0.48860251190291987 * x, 1.0925484305920792 * xy, -1.0925484305920792 * yz,
                      0.94617469575755997 * z2 - 0.31539156525251999, -1.0925484305920792 * xz,
                      0.54627421529603959 * x2 - 0.54627421529603959 * y2,
                      0.59004358992664352 * y * (-3.0 * x2 + y2), 2.8906114426405538 * xy * z,
                      0.45704579946446572 * y * (1.0 - 5.0 * z2), 0.3731763325901154 * z * (5.0 * z2 - 3.0),
                      0.45704579946446572 * x * (1.0 - 5.0 * z2), 1.4453057213202769 * z * (x2 - y2),
                      0.59004358992664352 * x * (-x2 + 3.0 * y2)], 1)
    h = torch.cat([feat, sh], 1)
    h = torch.relu(h @ torch.from_numpy(W1).T)
    h = torch.relu(h @ torch.from_numpy(W2).T)
    return torch.sigmoid(h @ torch.from_numpy(W3).T)[:, :3]


def rvq_torch(cb, idx, bias):
    """Ordered stage sum ((cb0[i0] + cb1[i1]) + cb2[i2]) + cb3[i3] + bias."""
    import torch
    c = torch.from_numpy(cb)
    ix = torch.from_numpy(idx.astype(np.int64))
    v = c[0][ix[:, 0]]
    for s in range(1, cb.shape[0]):
        v = v + c[s][ix[:, s]]
    return torch.from_numpy(np.asarray(bias, np.float32)) + v


def frame(scene, rows, workers: int, row_stride: int = 1, row_phase: int = 0):
    """Baseline frame of camera 0 on the tile rows `rows` (all rows: the whole
    frame): returns the outputs of the sampled pixels and stage wall times."""
    import multiprocessing as mp

    import torch

    from oracle import oracle as O
    sp = scene.spec
    cam = scene.cameras[0]
    W, H = cam.image_width, cam.image_height
    t = {}
    scales, rots, opac = scene.scales, scene.rotations, scene.opacity
    homo = scene.homotrans
    if sp.rvq:
        from nest_splat.scene import RVQ_BIAS, build_homotrans_np
        t0 = time.perf_counter()
        raw = {a: rvq_torch(scene.rvq_codebooks[a], scene.rvq_indices[a], RVQ_BIAS[a]) for a in RVQ_BIAS}
        scales = torch.exp(raw["scale"]).numpy()
        rots = torch.nn.functional.normalize(raw["rotation"], dim=1).numpy()
        opac = torch.sigmoid(raw["opacity"]).numpy()
        homo = build_homotrans_np(rots, scales, scene.means)
        t["rvq"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    pre = O.preprocess(scene.means, scales, rots, opac, cam.world_view_transform, cam.full_proj_transform, W, H)
    b = O.binning(pre, W, H)
    t["preprocess+binning"] = time.perf_counter() - t0
    gx = (W + BLOCK - 1) // BLOCK
    _STATE.update(W=W, H=H, gx=gx, ranges=b["ranges"], point_list=b["vals"], transmat=pre["transmat"].reshape(-1, 9),
                  xy=pre["xy"].reshape(-1, 2), normal_opacity=pre["normal_opacity"].reshape(-1, 4),
                  homotrans=np.ascontiguousarray(homo, np.float32).reshape(-1, 16),
                  ap=np.floor(np.asarray(scene.ap_level, np.float32).reshape(-1)).astype(np.int64))
    tiles = [ty * gx + tx for ty in rows for tx in range(gx)]
    t0 = time.perf_counter()
    if workers > 1:
        with mp.get_context("fork").Pool(workers) as pool:
            parts = pool.map(render_tile, tiles, chunksize=max(1, len(tiles) // (4 * workers)))
    else:
        parts = [render_tile(tl) for tl in tiles]
    t["render loop"] = time.perf_counter() - t0
    torch.set_num_threads(max(1, workers))
    grid = dict(L=sp.L, F=sp.F, S=sp.S, H=sp.base_res, offsets=np.asarray(scene.offsets, np.int64),
                table_t=torch.from_numpy(np.asarray(scene.table, np.float32)), contract=sp.contract,
                range=(float(sp.gridrange[0]), float(sp.gridrange[1])))
    t0 = time.perf_counter()
    # every accepted hit of the sample in one batch (chunks of 1M hits):
    # feature rows of the sampled pixels += w * query_feature(xyz)
    pix_all, others, hp_all, hx_all, hw_all, ha_all = [], [], [], [], [], []
    base = 0
    for (pix, oth, hp, hx, hw, ha, inside) in parts:
        local = np.full(BLOCK * BLOCK, -1, np.int64)
        local[np.nonzero(inside)[0]] = base + np.arange(int(inside.sum()))
        hp_all.append(local[hp])
        hx_all.append(hx)
        hw_all.append(hw)
        ha_all.append(ha)
        pix_all.append(pix)
        others.append(oth)
        base += int(inside.sum())
    pix_all = np.concatenate(pix_all)
    hp_all, hx_all = np.concatenate(hp_all), np.concatenate(hx_all)
    hw_all, ha_all = np.concatenate(hw_all), np.concatenate(ha_all)
    feat = torch.zeros((pix_all.size, sp.C), dtype=torch.float32)
    for c0 in range(0, hp_all.size, 1 << 20):
        sl = slice(c0, c0 + (1 << 20))
        enc = hash_encode_torch(hx_all[sl], ha_all[sl], grid)[:, :sp.C]
        if enc.shape[1] < sp.C:
            enc = torch.nn.functional.pad(enc, (0, sp.C - enc.shape[1]))
        feat.index_add_(0, torch.from_numpy(hp_all[sl]), enc * torch.from_numpy(hw_all[sl])[:, None])
    t["hash encode"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    dirs = O.ray_dirs(cam)[pix_all]
    rgb = mlp_torch(feat, dirs, scene.W1.astype(np.float32), scene.W2.astype(np.float32), scene.W3.astype(np.float32))
    alpha = np.concatenate([o[1] for o in others])
    rgb = torch.where(torch.from_numpy(alpha)[:, None] > 0, rgb, torch.zeros_like(rgb))
    if sum(sp.bg) > 0:
        rgb = rgb + (1 - torch.from_numpy(alpha))[:, None] * torch.tensor(sp.bg, dtype=torch.float32)
    t["mlp"] = time.perf_counter() - t0
    nr_sample = int(sum(int(b["ranges"][tl, 1]) - int(b["ranges"][tl, 0]) for tl in tiles))
    hits = int(sum(o[7].sum() for o in others))
    return dict(pix=pix_all, others=np.concatenate(others, 1), feat=feat.numpy(), rgb=rgb.numpy(), times=t,
                nr_total=b["num_rendered"], nr_sample=nr_sample, hits_sample=hits, tiles=len(tiles), gy=(H + 15) // 16,
                pixels=int(pix_all.size))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", default="cfg3")
    ap.add_argument("--row-stride", type=int, default=16)
    ap.add_argument("--workers", type=int, default=0)
    ap.add_argument("--gpu-hits", type=int, default=0, help="accepted hits of the whole frame (GPU), for the share")
    a = ap.parse_args()
    from nest_splat.scene import get_spec, make_scene
    workers = a.workers or len(os.sched_getaffinity(0))
    scene = make_scene(get_spec(a.config))
    gy = (scene.cameras[0].image_height + 15) // 16
    phase = a.row_stride // 2
    rows = [ty for ty in range(gy) if ty % a.row_stride == phase]
    t0 = time.perf_counter()
    r = frame(scene, rows, workers)
    wall = time.perf_counter() - t0
    t = r["times"]
    hits_total = a.gpu_hits or int(round(r["hits_sample"] * gy / max(1, len(rows))))
    share = (r["nr_sample"] + r["hits_sample"]) / max(1, r["nr_total"] + hits_total)
    pix_share = r["pixels"] / (scene.cameras[0].image_width * scene.cameras[0].image_height)
    frame_s = t.get("rvq", 0.0) + t["preprocess+binning"] + (t["render loop"] + t["hash encode"]) / share + \
        t["mlp"] / pix_share
    W, H = scene.cameras[0].image_width, scene.cameras[0].image_height
    print(json.dumps({"value": W * H / frame_s / 1e6, "unit": "Mpix/s", "cores": workers, "frame_s": frame_s,
                      "share": share, "pixel_share": pix_share, "rows": len(rows), "row_stride": a.row_stride,
                      "stage_s": {k: round(v, 3) for k, v in t.items()}, "wall_s": wall}))


if __name__ == "__main__":
    main()
