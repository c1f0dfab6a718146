#!/usr/bin/env python3
"""Headline benchmark: rendered Mpix/s of the forward path (preprocess ->
binning -> tile render with in-loop hash lookup -> MLP decode) on the
1M-splat, 1600x1064, 16-level hash-textured unbounded scene, with the render
kernel's HBM roofline fraction and the benchmark's CPU path (NumPy per-pixel loop,
torch-CPU hash encode, MLP and RVQ) timed on this host.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--config cfg3]

--config picks the workload: cfg1 (2k splats, 128x128), cfg2 (100k splats,
800x800), cfg3 (the default and the metric: 1M splats, 1600x1064), cfg4
(500k RVQ-compressed splats, the decode inside the timed frame), cfg5 (4M
splats, all eight 1920x1080 cameras per step).

Prints one JSON line.  One process drives one GPU; --gpus above 1 exits with a
message (frames shard by camera or by tile band across processes).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "nest-splatting_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "rendered Mpix/s (raster+hash+MLP), 1M splats @1600x1064; % HBM roofline"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def render_algorithmic_bytes(NR: int, hits: int, HW: int, L: int, F: int, e: int, C: int) -> int:
    """Logical bytes of one render launch, cache hits included: 104 B per
    staged tile/splat pair, L*8*F*e B of hash gathers per accepted hit,
    (4C + 56) B of outputs per pixel (colour map + 14 allmap channels)."""
    return 104 * NR + L * 8 * F * e * hits + HW * (4 * C + 56)


def render_compulsory_bound(P: int, NR: int, HW: int, table_bytes: int, C: int) -> int:
    """Upper bound of the bytes one render launch must exchange with HBM once:
    every splat's 128-B record, the 4-B point list entry per pair, the whole
    table (the bound takes every entry as touched), the outputs."""
    return 128 * P + 4 * NR + table_bytes + HW * (4 * C + 56)


# What bounds the render kernel, from its counters (TA busy, L1 accesses per
# clock, VALU share): the 16-byte table gathers' vector-L1 address and tag
# rate and the latency of the gathers that miss L2.
RENDER_LIMITER = ("the lookup drains' instruction stream: VALU issue ~0.63 and the texture addresser ~0.75 busy on "
                  "the 1M-splat frame (one L1 tag access per CU clock); with every gather L1-resident the render "
                  "takes 0.90x its time, without the drains 0.24x; HBM traffic is the counter-measured fetch + "
                  "write")


def load_counters(path: str) -> dict:
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def cpu_baseline(config: str, gpu_hits_total: int, row_stride: int, threads: int):
    """The CPU path of the benchmark definition, timed on this host: a NumPy
    transcription of the per-pixel render loop (parallel over tiles with a
    pool of `threads` processes), torch-CPU hash encode of the accepted hits,
    torch-CPU MLP and RVQ, with preprocess and binning from the C oracle
    (oracle/cpu_baseline.py).  It runs in a child process that touches no
    GPU, on every row_stride-th tile row, and is scaled to a frame by the
    sample's share of tile/splat pairs plus hits (render loop and hash encode)
    and of pixels (MLP)."""
    import subprocess
    cmd = [sys.executable, "-m", "oracle.cpu_baseline", "--config", config, "--row-stride", str(row_stride),
           "--workers", str(threads), "--gpu-hits", str(gpu_hits_total)]
    r = subprocess.run(cmd, cwd=ROOT, capture_output=True, text=True, timeout=900)
    if r.returncode != 0:
        raise RuntimeError(f"cpu baseline failed ({r.returncode}): {r.stderr[-2000:]}")
    res = json.loads(r.stdout.strip().splitlines()[-1])
    st = res["stage_s"]
    parts = "; ".join(f"{k} {v:.2f} s" for k, v in st.items())
    return {
        "value": res["value"],
        "unit": "Mpix/s",
        "cores": res["cores"],
        "kind": "port",
        "sample": (f"NumPy per-pixel loop over {res['rows']} of every {row_stride} tile rows ({res['cores']} worker "
                   f"processes) + torch-CPU hash encode, MLP{' and RVQ' if 'rvq' in st else ''} "
                   f"({res['cores']} threads), C-oracle preprocess and binning (1 thread): {parts}; scaled by the "
                   f"sample's {res['share']:.4f} share of pairs+hits and {res['pixel_share']:.4f} of pixels; "
                   f"extrapolated frame {res['frame_s']:.1f} s"),
        "frame_s": res["frame_s"],
    }


def summarize_pmc(fetch_dir: str, write_dir: str, out_path: str, kernel: str = "render_kernel") -> dict:
    """Reduce two rocprofv3 --pmc runs (FETCH_SIZE, then WRITE_SIZE, both with
    --copy-calibration-mb) to HBM bytes per launch of the kernels whose name
    contains `kernel`.  Each counter is scaled by bytes-moved /
    counter-reading of the largest plain copy kernel (__amd_rocclr_copyBuffer)
    in the same run."""
    import csv
    import glob

    def rows(d):
        out = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            out += list(csv.DictReader(open(f)))
        return out

    res = {}
    for tag, d, counter in (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        rs = [r for r in rows(d) if r["Counter_Name"] == counter]
        copies = [float(r["Counter_Value"]) for r in rs if "copyBuffer" in r["Kernel_Name"]]
        render = [float(r["Counter_Value"]) for r in rs if kernel in r["Kernel_Name"]]
        if not copies or not render:
            raise SystemExit(f"no copy/render rows for {counter} under {d}")
        copy_kib = max(copies)
        res[f"{tag}_copy_counter_kib"] = copy_kib
        res[f"{tag}_render_counter_kib"] = sum(render) / len(render)
        res[f"{tag}_launches"] = len(render)
    return res


def finish_traffic(res: dict, copy_mib: int, out_path: str) -> dict:
    moved_kib = copy_mib * 1024.0
    res["copy_mib"] = copy_mib
    res["fetch_scale"] = moved_kib / res["fetch_copy_counter_kib"]
    res["write_scale"] = moved_kib / res["write_copy_counter_kib"]
    res["render_fetch_bytes"] = res["fetch_render_counter_kib"] * 1024 * res["fetch_scale"]
    res["render_write_bytes"] = res["write_render_counter_kib"] * 1024 * res["write_scale"]
    res["render_bytes_per_launch"] = int(res["render_fetch_bytes"] + res["render_write_bytes"])
    with open(out_path, "w") as f:
        json.dump(res, f, indent=1)
    return res


def time_aux_kernels(K, spec, scene, table, dev):
    """HIP-event times of the RVQ decode (the 4-stage, 4096-entry compressed
    scene: scale, rotation and opacity in one launch, 52 algorithmic bytes per
    splat; at its 500k splats and at 4M) and of the GridEncoder forward (1M
    points of this scene's grid, B·(12 + L·8·F·e + L·F·e) algorithmic bytes),
    K launches each."""
    import numpy as np
    import torch

    from gridencoder.grid import grid_encode_forward
    from nest_splat import rvq
    from nest_splat.scene import RVQ_BIAS, get_spec, make_scene

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(K):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / K

    res = {}
    rs = get_spec("cfg4", P=500_000)
    rsc = make_scene(rs)
    for P in (500_000, 4_000_000):
        # the compressed scene's codebooks; 4M splats repeat its indices 8 times
        reps = P // rs.P
        idx = {a: np.tile(rsc.rvq_indices[a], (reps, 1)) for a in rsc.rvq_indices}
        att = rvq.RVQAttributes.from_numpy(rsc.rvq_codebooks, idx, RVQ_BIAS, dev)
        ms = timed(lambda: att.decode())
        nbytes = 52 * P
        res[f"rvq_decode_{P // 1000}k"] = {"ms": round(ms, 4), "splats": P, "algorithmic_bytes": nbytes,
                                           "GB/s": round(nbytes / ms / 1e6, 1),
                                           "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
    B = 1_000_000
    pts = torch.rand((B, 3), generator=torch.Generator(device=dev).manual_seed(3), device=dev)
    offs = np.asarray(scene.offsets, np.int64)
    ms = timed(lambda: grid_encode_forward(pts, table, offs, float(2.0 ** spec.S), spec.base_res))
    e = scene.table.dtype.itemsize
    nbytes = B * (12 + spec.L * 8 * spec.F * e + spec.L * spec.F * e)
    res["grid_encode"] = {"ms": round(ms, 4), "points": B, "algorithmic_bytes": nbytes,
                          "GB/s": round(nbytes / ms / 1e6, 1), "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4)}
    log(f"[bench] rvq decode {res['rvq_decode_500k']['ms']} / {res['rvq_decode_4000k']['ms']} ms (500k / 4M splats), "
        f"grid encode {res['grid_encode']['ms']} ms")
    return res


def time_modes(K, spec, scene, settings, means, opac, scales, rots, homo, ap_level, table, mlp, M, bg, dev,
               hyb=10):
    """Render modes 4, 6, 7, 12, 13 and 14 on the benchmark frame: the first `hyb` of
    the 16 levels become per-splat feature rows, the last 16 - hyb levels the
    grid (the scene's own tables of those levels, base resolution of level
    hyb); mode 6 blends 64-channel rows half and half with the scene's whole
    16-level grid.  Mode 12/13 rows carry a blend weight uniform in [0.15, 1): 59% of
    the splats take mode 13's inference fast path (weight > 0.5), 12% mode
    12's (weight >= 0.9); none skip mode 14's grid (weight < 0.1).  Mode 7
    blends all 16 row levels with the grid.  Modes 4, 7, 12 and 14 also time
    their backward.  Returns per mode the mean render-kernel
    and frame (render + MLP) milliseconds over K frames."""
    import numpy as np
    import torch

    from nest_splat import _lib as L
    from nest_splat import rasterizer as rz
    F, Lt = spec.F, spec.L
    gl = Lt - hyb
    offs = np.asarray(scene.offsets, np.int64)
    sub_offsets = offs[hyb:] - offs[hyb]
    sub_table = table[int(offs[hyb]):int(offs[Lt])]
    sub_base = int(round(2.0 ** (hyb * spec.S) * spec.base_res))
    rng = np.random.default_rng(1)
    tdim = Lt * F
    rows = (rng.standard_normal((spec.P, tdim + 1)) * 0.1).astype(np.float32)
    rows[:, tdim] = rng.uniform(0.15, 1.0, spec.P).astype(np.float32)
    rows13 = torch.from_numpy(rows).to(dev)
    rows4 = rows13[:, :hyb * F].contiguous()
    rows14 = torch.cat([rows4, rows13[:, tdim:]], dim=1).contiguous()
    rows6 = rows13[:, :tdim].contiguous()
    cases = {"cat(4)": (4, rows4, 0), "adaptive(6)": (6, rows6, 0), "adaptive_add(7)": (7, rows13, Lt),
             "adaptive_cat(12) training": (12, rows13, Lt),
             "adaptive_cat(12) inference": (12 | 0x100, rows13, Lt),
             "adaptive_cat_fast(13) training": (13, rows13, Lt),
             "adaptive_cat_fast(13) inference": (13 | 0x100, rows13, Lt),
             "adaptive_zero(14) training": (14, rows14, Lt),
             "adaptive_zero(14) inference": (14 | 0x100, rows14, Lt)}
    res_ms = {}
    for name, (mode, rows_t, total) in cases.items():
        if mode == 6:
            grid = rz.HashGridDesc(Lt, F, spec.S, spec.base_res, table, offs, np.asarray(spec.gridrange, np.float32),
                                   render_mode=6)
        else:
            # mode 7 blends all 16 levels of the row with the 6-level grid (no coarse levels)
            grid = rz.HashGridDesc(gl, F, spec.S, sub_base, sub_table, sub_offsets,
                                   np.asarray(spec.gridrange, np.float32), render_mode=mode,
                                   hybrid_levels=0 if mode == 7 else hyb, total_levels=total)

        def frame(tm=None):
            res = rz.rasterize_forward(settings, grid, means, opac, scales, rots, homotrans=homo, ap_level=ap_level,
                                       colors_precomp=rows_t, channels=spec.C,
                                       timing=tm if tm is not None else False)
            return res, mlp.decode_image(res.color, M, alpha=res.others[1], bg=bg)

        frame()
        torch.cuda.synchronize()
        tms = [L.new_timing(True) for _ in range(K)]
        t0 = time.perf_counter()
        for k in range(K):
            frame(tms[k])
        torch.cuda.synchronize()
        frame_ms = (time.perf_counter() - t0) / K * 1e3
        render_ms = float(np.mean([L.timing_read(tm)["render"] for tm in tms]))
        for tm in tms:
            L.timing_release(tm)
        res_ms[name] = {"render_ms": round(render_ms, 4), "frame_ms": round(frame_ms, 4)}
        log(f"[bench] {name}: render {render_ms:.3f} ms, frame {frame_ms:.3f} ms")
        if mode in (4, 7, 12, 14):
            # training step of modes 4, 7, 12 and 14: the backward of the last frame,
            # every grid level active, random output gradients
            res, _ = frame()
            gen = torch.Generator(device=dev).manual_seed(0)
            dcol = torch.randn(tuple(res.color.shape), generator=gen, device=dev)
            doth = torch.randn(tuple(res.others.shape), generator=gen, device=dev)

            def bwd():
                return rz.rasterize_backward(settings, grid, res, means, opac, scales, rots, dcol, doth,
                                             homotrans=homo, ap_level=ap_level, colors_precomp=rows_t,
                                             channels=spec.C)
            bwd()
            torch.cuda.synchronize()
            b0 = time.perf_counter()
            for _ in range(K):
                bwd()
            torch.cuda.synchronize()
            res_ms[name]["backward_ms"] = round((time.perf_counter() - b0) / K * 1e3, 3)
            log(f"[bench] {name}: backward {res_ms[name]['backward_ms']} ms")
    # hybrid SH modes 8-10: a one-level 3-channel grid at the finest resolution
    # (2048, 2^21 entries) and rows of 3 raw SH colours or 48 coefficients; the
    # image is the 3 (or 48) blended channels, no MLP
    gen = torch.Generator(device=dev).manual_seed(2)
    htab = (torch.rand((1 << 21, 3), generator=gen, device=dev) - 0.5) * 0.2
    hgrid_args = (1, 3, 0.0, 2048, htab, np.array([0, 1 << 21], np.int64), np.asarray(spec.gridrange, np.float32))
    raw = torch.randn((spec.P, 3), generator=gen, device=dev)
    coeffs = torch.randn((spec.P, 48), generator=gen, device=dev) * 0.3
    for name, mode, rows_t in (("hybrid_SH(8)", 8, raw), ("hybrid_SH_post(9)", 9, coeffs), ("hybrid_SH_raw(10)", 10, raw)):
        grid = rz.HashGridDesc(*hgrid_args, render_mode=mode)
        C = 48 if mode == 9 else 3

        def hframe(tm=None):
            return rz.rasterize_forward(settings, grid, means, opac, scales, rots, homotrans=homo, ap_level=ap_level,
                                        colors_precomp=rows_t, channels=C, timing=tm if tm is not None else False)

        hframe()
        torch.cuda.synchronize()
        tms = [L.new_timing(True) for _ in range(K)]
        t0 = time.perf_counter()
        for k in range(K):
            hframe(tms[k])
        torch.cuda.synchronize()
        frame_ms = (time.perf_counter() - t0) / K * 1e3
        render_ms = float(np.mean([L.timing_read(tm)["render"] for tm in tms]))
        for tm in tms:
            L.timing_release(tm)
        res_ms[name] = {"render_ms": round(render_ms, 4), "frame_ms": round(frame_ms, 4)}
        log(f"[bench] {name}: render {render_ms:.3f} ms, frame {frame_ms:.3f} ms")
    return res_ms


class Workload:
    """The timed step of one config: its device inputs and a step(timings)
    closure that renders every camera of the config once (cfg4: decodes the
    RVQ attributes first) and decodes the feature maps with the MLP."""

    def __init__(self, spec, scene, dev):
        import numpy as np
        import torch

        from nest_splat import rasterizer as rz
        from nest_splat.camera import view_ray_matrix
        from nest_splat.mlp import NestMLP

        self.spec, self.scene = spec, scene
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
        self.means, self.opac, self.scales, self.rots = t(scene.means), t(scene.opacity), t(scene.scales), \
            t(scene.rotations)
        self.homo, self.ap_level, self.table = t(scene.homotrans), t(scene.ap_level), t(scene.table)
        self.grid = rz.HashGridDesc(spec.L, spec.F, spec.S, spec.base_res, self.table, scene.offsets,
                                    np.asarray(spec.gridrange, np.float32))
        self.mlp = NestMLP(spec.C, spec.mlp_width, spec.mlp_dtype, scene.W1, scene.W2, scene.W3).to(dev)
        self.bg = torch.tensor(spec.bg, dtype=torch.float32) if sum(spec.bg) > 0 else None
        self.cams = scene.cameras
        self.settings = [rz.make_settings(c.image_height, c.image_width, c.tanfovx, c.tanfovy, c.world_view_transform,
                                          c.full_proj_transform, c.camera_center, if_contract=spec.contract)
                         for c in self.cams]
        self.rays = [view_ray_matrix(c) for c in self.cams]
        self.rvq = None
        if spec.rvq:
            from nest_splat.rvq import RVQAttributes
            from nest_splat.scene import RVQ_BIAS
            self.rvq = RVQAttributes.from_numpy(scene.rvq_codebooks, scene.rvq_indices, RVQ_BIAS, dev)
        self.pixels = sum(c.image_width * c.image_height for c in self.cams)
        self.mlp_events = []  # (start, stop) HIP events around each timed MLP decode

    def step(self, timings=None):
        """One step; timings: a list with one nest_timing per camera, or None."""
        import torch

        from nest_splat import rasterizer as rz
        means, opac, scales, rots, homo = self.means, self.opac, self.scales, self.rots, self.homo
        if self.rvq is not None:
            # compressed attributes: decode (exp / normalise / sigmoid fused) and
            # rebuild homotrans from the decoded rotation and scale, as the
            # reference rebuilds it every frame (get_homotrans)
            dec = self.rvq.decode()
            scales, rots, opac = dec["scale"], dec["rotation"], dec["opacity"]
            homo = rz.build_homotrans(rots, scales, means)
        out = []
        for k, (st, M) in enumerate(zip(self.settings, self.rays)):
            tm = timings[k] if timings is not None else False
            res = rz.rasterize_forward(st, self.grid, means, opac, scales, rots, homotrans=homo,
                                       ap_level=self.ap_level, channels=self.spec.C, timing=tm)
            ev = None
            if timings is not None:
                ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                ev[0].record()
            rgb = self.mlp.decode_image(res.color, M, alpha=res.others[1], bg=self.bg)
            if ev is not None:
                ev[1].record()
                self.mlp_events.append(ev)
            out.append((res, rgb))
        return out


def describe(spec) -> str:
    layout = {"cube": "centres uniform in [-1,1]^3", "shell": "noisy unit sphere shell",
              "ball_unbounded": "70% in a unit ball and 30% out to r=20 (contracted)",
              "shells": "5 noisy concentric shells (r 0.5-2.5)"}[spec.layout]
    cams = f"{spec.n_cams} cameras at " if spec.n_cams > 1 else ""
    rvq = (f", scale/rotation/opacity as {spec.rvq_stages}-stage RVQ codes into {spec.rvq_codebook}-entry codebooks "
           f"decoded inside the step") if spec.rvq else ""
    return (f"{spec.name}: {spec.P} 2D surfels, {layout}{rvq}; {cams}{spec.W}x{spec.H}, hash grid L={spec.L} "
            f"F={spec.F} T=2^{spec.log2T} {spec.table_dtype}, MLP {spec.C + 16}-{spec.mlp_width}-{spec.mlp_width}-3 "
            f"{spec.mlp_dtype}")


def main():
    if len(sys.argv) > 1 and sys.argv[1] == "--pmc-summary":
        # python bench.py --pmc-summary FETCH_DIR WRITE_DIR COPY_MIB OUT.json [KERNEL_SUBSTRING]
        fetch_dir, write_dir, copy_mib, out_path = sys.argv[2:6]
        kern = sys.argv[6] if len(sys.argv) > 6 else "render_kernel"
        r = finish_traffic(summarize_pmc(fetch_dir, write_dir, out_path, kern), int(copy_mib), out_path)
        print(json.dumps(r))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="cfg3", choices=["cfg1", "cfg2", "cfg3", "cfg4", "cfg5"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-row-stride", type=int, default=0,
                    help="CPU baseline: render every k-th tile row (0: per-config default)")
    ap.add_argument("--traffic", default=None,
                    help="JSON with counter-measured HBM bytes per render launch (from rocprofv3 --pmc); default "
                         "profiles/render_traffic_<config>.json")
    ap.add_argument("--counters", default=None,
                    help="JSON with the render kernel's L1 counters (TCP_TOTAL_CACHE_ACCESSES, kernel cycles); "
                         "default profiles/render_counters_<config>.json")
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="before the frames, copy this many MiB device-to-device (a plain copy kernel of known "
                         "size whose FETCH_SIZE / WRITE_SIZE scale the render kernel's counters)")
    ap.add_argument("--modes", type=int, default=0, metavar="K",
                    help="after the timed frames, time K frames of each other render mode (4 cat, 7 adaptive_add, 12 "
                         "adaptive_cat, 13 adaptive_cat_fast and 14 adaptive_zero, training and inference) on the same splats: per-splat rows of the "
                         "first 10 levels, a grid of the last 6, and report modes_ms, with K backward passes of modes 4, 7, 12 and 14; "
                         "then the hybrid SH modes 8, 9 and 10 over a one-level 3-channel grid "
                         "(not part of the metric)")
    ap.add_argument("--kernels", type=int, default=0, metavar="K",
                    help="after the timed frames, time K launches of the other hot-path kernels on their own: the RVQ "
                         "decode of the 500k-splat compressed scene and the GridEncoder forward of 1M points on this "
                         "grid; reports aux_kernels with algorithmic GB/s (not part of the metric)")
    ap.add_argument("--record", type=int, default=0, metavar="K",
                    help="after the timed frames, time K frames with record_transmittance=True (the densification "
                         "statistic's extra pass) and report record_ms: render stage and frame with and without it "
                         "(not part of the metric)")
    ap.add_argument("--backward", type=int, default=0, metavar="K",
                    help="after the timed forward frames, time K backward passes (nest_backward) of the last frame "
                         "with random output gradients and report backward_ms (not part of the metric)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark drives exactly one GPU per process; multi-GPU figures are not "
                                   "produced (frames shard by camera or tile band across processes)",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    import numpy as np
    import torch

    from nest_splat import _lib as L
    from nest_splat import rasterizer as rz
    from nest_splat.scene import get_spec, make_scene

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    L.lib()
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    spec = get_spec(args.config)
    scene = make_scene(spec)
    log(f"[bench] scene {spec.name}: {spec.P} splats, {spec.n_cams} x {spec.W}x{spec.H}, table "
        f"{scene.table.nbytes / 2**20:.0f} MiB ({time.perf_counter() - t0:.1f} s)")
    wl = Workload(spec, scene, dev)
    ncam = len(wl.cams)

    if args.copy_calibration_mb > 0:
        n = args.copy_calibration_mb * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy calibration: 3 x {args.copy_calibration_mb} MiB device copies")
        del src, dst
    for i in range(args.warmup):
        frames = wl.step()
    torch.cuda.synchronize()
    log(f"[bench] warmup done ({args.warmup} steps)")
    tms = [[L.new_timing(True) for _ in range(ncam)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for k in range(args.steps):
        frames = wl.step(tms[k])
    torch.cuda.synchronize()
    t_end = time.perf_counter()
    stages = [L.timing_read(tm) for row in tms for tm in row]
    for row in tms:
        for tm in row:
            L.timing_release(tm)
    elapsed = t_end - t_start
    ms_per_step = elapsed / args.steps * 1e3
    mpix = wl.pixels * args.steps / elapsed / 1e6
    log(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step, {mpix:.1f} Mpix/s")

    HW = spec.W * spec.H
    hits_total = [int(res.others[7].double().sum().item()) for res, _ in frames]
    NRs = [res.num_rendered for res, _ in frames]
    render_ms = float(np.mean([s["render"] for s in stages]))
    stage_ms = {k: float(np.mean([s[k] for s in stages])) for k in stages[0]}
    stage_ms["mlp"] = float(np.mean([a.elapsed_time(b) for a, b in wl.mlp_events]))
    e = scene.table.dtype.itemsize
    alg = float(np.mean([render_algorithmic_bytes(nr, h, HW, spec.L, spec.F, e, spec.C)
                         for nr, h in zip(NRs, hits_total)]))
    comp = float(np.mean([render_compulsory_bound(spec.P, nr, HW, scene.table.nbytes, spec.C) for nr in NRs]))
    tpath = args.traffic or os.path.join(ROOT, "profiles", f"render_traffic_{spec.name}.json")
    traffic = load_counters(tpath).get("render_bytes_per_launch")
    cpath = args.counters or os.path.join(ROOT, "profiles", f"render_counters_{spec.name}.json")
    ctr = load_counters(cpath)
    achieved = traffic / (render_ms * 1e-3) / 1e9 if traffic else None
    roofline = {"bound": "hbm", "kernel": "render_kernel (tile compositing + hash gathers)",
                "achieved": round(achieved, 1) if achieved else None, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None, "traffic": traffic,
                "traffic_source": os.path.relpath(tpath, ROOT) if traffic else None,
                "render_ms": round(render_ms, 4),
                "algorithmic_bytes": int(alg),
                "algorithmic_GBps_cache_inclusive": round(alg / (render_ms * 1e-3) / 1e9, 1),
                "compulsory_bytes_bound": int(comp),
                "limiter": RENDER_LIMITER}
    if ctr.get("TCP_TOTAL_CACHE_ACCESSES_sum") and ctr.get("kernel_cycles"):
        roofline["l1_tag_accesses_per_cu_clock"] = round(
            ctr["TCP_TOTAL_CACHE_ACCESSES_sum"] / (ctr.get("cus", 256) * ctr["kernel_cycles"]), 3)
    if ctr.get("TA_BUSY_avr") and ctr.get("kernel_cycles"):
        roofline["ta_busy"] = round(ctr["TA_BUSY_avr"] / ctr["kernel_cycles"], 3)
    if ctr.get("SQ_INSTS_VALU") and ctr.get("kernel_cycles"):
        # a wave64 VALU instruction occupies its 16-lane SIMD for 4 cycles; 4 SIMDs per CU
        roofline["valu_issue"] = round(4 * ctr["SQ_INSTS_VALU"] / (4 * ctr.get("cus", 256) * ctr["kernel_cycles"]), 3)
    out = {
        "metric": METRIC,
        "value": round(mpix, 3),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded scene generator, random-init hash table and Xavier MLP weights)",
        "config": {"workload": describe(spec), "splats": spec.P, "width": spec.W, "height": spec.H,
                   "cameras": ncam, "num_rendered": int(np.mean(NRs)),
                   "hits_per_pixel": round(sum(hits_total) / (HW * ncam), 3)},
        "frames_per_s": round(1e3 * ncam / ms_per_step, 3),
        "stages_ms": {k: round(v, 4) for k, v in stage_ms.items()},
        "roofline": roofline,
        "cpu_baseline": None,
    }
    res, rgb = frames[-1]
    means, opac, scales, rots, homo, ap_level, table = wl.means, wl.opac, wl.scales, wl.rots, wl.homo, wl.ap_level, \
        wl.table
    settings, grid, mlp, bg = wl.settings[-1], wl.grid, wl.mlp, wl.bg
    if (args.modes or args.backward) and spec.rvq:
        raise SystemExit("--modes / --backward run on the uncompressed configs")
    if args.modes > 0:
        out["modes_ms"] = time_modes(args.modes, spec, scene, settings, means, opac, scales, rots, homo, ap_level,
                                     table, mlp, wl.rays[-1], bg, dev)
    if args.kernels > 0:
        out["aux_kernels"] = time_aux_kernels(args.kernels, spec, scene, table, dev)
    if args.record > 0:
        rec_ms = {}
        for rec in (False, True):
            def rframe(tm):
                r = rz.rasterize_forward(settings, grid, means, opac, scales, rots, homotrans=homo, ap_level=ap_level,
                                         channels=spec.C, timing=tm, record_transmittance=rec)
                return r, mlp.decode_image(r.color, wl.rays[-1], alpha=r.others[1], bg=bg)
            rframe(False)
            torch.cuda.synchronize()
            rtms = [L.new_timing(True) for _ in range(args.record)]
            r0 = time.perf_counter()
            for k in range(args.record):
                rframe(rtms[k])
            torch.cuda.synchronize()
            fr = (time.perf_counter() - r0) / args.record * 1e3
            rr = float(np.mean([L.timing_read(tm)["render"] for tm in rtms]))
            for tm in rtms:
                L.timing_release(tm)
            rec_ms["with_record" if rec else "without"] = {"render_ms": round(rr, 4), "frame_ms": round(fr, 4)}
            log(f"[bench] record_transmittance={rec}: render stage {rr:.3f} ms, frame {fr:.3f} ms")
        out["record_ms"] = rec_ms
    if args.backward > 0:
        gen = torch.Generator(device=dev).manual_seed(0)
        dcol = torch.randn(tuple(res.color.shape), generator=gen, device=dev)
        doth = torch.randn(tuple(res.others.shape), generator=gen, device=dev)
        bwd = lambda: rz.rasterize_backward(settings, grid, res, means, opac, scales, rots, dcol, doth, homotrans=homo,
                                            ap_level=ap_level, channels=spec.C)
        bwd()
        torch.cuda.synchronize()
        b0 = time.perf_counter()
        for _ in range(args.backward):
            bwd()
        torch.cuda.synchronize()
        out["backward_ms"] = round((time.perf_counter() - b0) / args.backward * 1e3, 3)
        log(f"[bench] backward: {out['backward_ms']} ms")
    if not args.no_cpu_baseline:
        # camera 0 of the config (the rate per camera is the rate per frame)
        threads = len(os.sched_getaffinity(0))
        stride = args.cpu_row_stride or {"cfg1": 1, "cfg2": 1, "cfg3": 16, "cfg4": 16, "cfg5": 34}[spec.name]
        log(f"[bench] cpu baseline on {threads} cores ...")
        cb = cpu_baseline(spec.name, hits_total[0], stride, threads)
        out["cpu_baseline"] = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in cb.items() if k != "frame_s"}
        if spec.name == "cfg1" and threads > 1:
            one = cpu_baseline(spec.name, hits_total[0], stride, 1)
            out["cpu_baseline"]["value_1_core"] = round(one["value"], 6)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
