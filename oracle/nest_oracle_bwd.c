/*
 * nest_oracle_bwd.c -- CPU oracle for the backward pass (training) of render
 * mode 0 with the Gaussian kernel, and of the standalone GridEncoder.
 *
 * TEST INFRASTRUCTURE ONLY, like nest_oracle.c, at whose end this file is
 * included (one translation unit, so it shares that file's helpers and float
 * contract).  Reference text restated here:
 *   CR/hashgrid.h:53-299          query_feature<true, C, F>
 *   CR/backward.cu:445-2049       renderCUDAsurfelBackward, mode 0, kernel_type 0
 *   CR/backward.cu:20-140         computeColorFromSH backward
 *   CR/backward.cu:2056-2274      compute_transmat_aabb, preprocessCUDA
 *   CR/auxiliary.h:115-160, :244-297  transformVec4x3Transpose, dnormvdv,
 *                                 quat_to_rotmat_vjp, scale_to_mat
 *   GE/src/gridencoder.cu:196-242, :245-366  dy_dx, kernel_grid_backward,
 *                                 kernel_input_backward
 *
 * The reference accumulates every per-splat and per-table-entry gradient with
 * atomicAdd, in an order the hardware picks.  Here the same sums run
 * sequentially (tiles in order, pixels row-major inside a tile, splats back to
 * front), so the GPU is compared against these values within a tolerance.
 * The per-pixel arithmetic follows the reference expression by expression,
 * left to right, without contraction; double literals follow C's promotion
 * (a float product stays a float product).
 *
 * Deliberate fidelity to the reference where it is not the exact derivative
 * of its own forward (documented with the functions below): the preprocess
 * backward rebuilds T with scale modifier 1 and differentiates the screen
 * centre with the cutoff-3 vector (9, 9, -1) while the forward uses 16; the
 * normal normalisation is differentiated as (g - (g.n) n / |n|) / |n|; the
 * contraction enters dL/dxyz only through the scalar grad_scale; opacity gets
 * G * dL/dalpha also where alpha was clamped to 0.99; with beta > 0 the
 * position terms use -G' s with the activated G' where the chain rule has the
 * raw -g s (CR/backward.cu:1910-1913, :1977); grad_means2D is replaced by the
 * densification statistic of CR/backward.cu:2269-2271.
 */

/* ------------------------------------------------------------------ */
/* hash grid backward: CR/hashgrid.h:53-299                             */
/* ------------------------------------------------------------------ */

/* query_feature<true, C, F>: recomputes feat[C] (as the forward), adds
 * w * grad_feat[l*F + ch] to dtable at every corner of every queried level,
 * and returns dL/dxyz = sum over levels and channels of grad_feat * dy/dxyz,
 * dy/dxyz being the trilinear (or smoothstep) derivative scaled by
 * scale * grad_scale (hashgrid.h:213-299).  Out-of-bounds points leave
 * feat = 0 and dxyz = 0 and touch no table entry. */
static void qf_backward(const or_grid *G, const float xyz[3], uint32_t ap, int C, const float *grad_feat,
                        float *feat, float *dtable, float dxyz[3])
{
    const int F = G->F;
    for (int c = 0; c < C; c++) feat[c] = 0.0f;
    dxyz[0] = dxyz[1] = dxyz[2] = 0.0f;
    float u[3];
    if (grid_normalise(G, xyz, u)) return;
    /* grad_scale of hashgrid.h:72-97 */
    float grad_scale;
    if (!G->contract) {
        grad_scale = 1.0f / (G->vmax - G->vmin);
    } else {
        float vmid = (G->vmax + G->vmin) * 0.5f;
        float inv = 1.0f / ((G->vmax - G->vmin) * 0.5f);
        float i0 = (xyz[0] - vmid) * inv, i1 = (xyz[1] - vmid) * inv, i2 = (xyz[2] - vmid) * inv;
        float norm = sqrtf(i0 * i0 + i1 * i1 + i2 * i2);
        float inv_norm = 1.0f / norm;
        float st = (norm <= 1.0f) ? 1.0f : (2.0f - inv_norm) * inv_norm;
        grad_scale = inv * st * 0.25f;
    }
    const uint32_t max_level = ap < (uint32_t)G->L ? ap : (uint32_t)G->L;
    float lpos[64][3], lder[64][3];
    uint32_t lg[64][3];
    for (uint32_t l = 0; l < max_level; l++) {
        uint32_t hsize = (uint32_t)(G->offsets[l + 1] - G->offsets[l]);
        float scale; uint32_t res;
        or_level_scale(G->S, G->H, (int)l, &scale, &res);
        size_t base = (size_t)(uint32_t)G->offsets[l] * (size_t)F;
        for (int d = 0; d < 3; d++) {
            float pos = u[d] * scale + (G->align_corners ? 0.0f : 0.5f);
            lg[l][d] = f2u_sat(floorf(pos));
            pos = pos - (float)lg[l][d];
            if (G->interp == 1) {
                lder[l][d] = 6.0f * pos * (1.0f - pos);
                pos = pos * pos * (3.0f - 2.0f * pos);
            } else {
                lder[l][d] = 1.0f;
            }
            lpos[l][d] = pos;
        }
        for (uint32_t corner = 0; corner < 8; corner++) {
            float w = 1.0f;
            uint32_t q[3];
            for (int d = 0; d < 3; d++) {
                if ((corner & (1u << d)) == 0) { w *= 1 - lpos[l][d]; q[d] = lg[l][d]; }
                else { w *= lpos[l][d]; q[d] = lg[l][d] + 1u; }
            }
            size_t e = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
            for (int ch = 0; ch < F; ch++) {
                feat[l * F + ch] = fmaf(w, table_at(G, e + ch), feat[l * F + ch]);
                dtable[e + ch] += w * grad_feat[l * F + ch];
            }
        }
    }
    /* dy/dxyz per level, dimension and channel (hashgrid.h:213-281) */
    float dydx[3][256];
    for (uint32_t l = 0; l < max_level; l++) {
        uint32_t hsize = (uint32_t)(G->offsets[l + 1] - G->offsets[l]);
        float scale; uint32_t res;
        or_level_scale(G->S, G->H, (int)l, &scale, &res);
        size_t base = (size_t)(uint32_t)G->offsets[l] * (size_t)F;
        for (int gd = 0; gd < 3; gd++) {
            float rg[16];
            for (int ch = 0; ch < F; ch++) rg[ch] = 0.0f;
            for (uint32_t idx = 0; idx < 4; idx++) {
                float w = scale * grad_scale;
                uint32_t q[3];
                for (int nd = 0; nd < 2; nd++) {
                    const int d = (nd >= gd) ? nd + 1 : nd;
                    if ((idx & (1u << nd)) == 0) { w *= 1 - lpos[l][d]; q[d] = lg[l][d]; }
                    else { w *= lpos[l][d]; q[d] = lg[l][d] + 1u; }
                }
                q[gd] = lg[l][gd];
                size_t el = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
                q[gd] = lg[l][gd] + 1u;
                size_t er = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
                for (int ch = 0; ch < F; ch++)
                    rg[ch] += w * (table_at(G, er + ch) - table_at(G, el + ch)) * lder[l][gd];
            }
            for (int ch = 0; ch < F; ch++) dydx[gd][l * F + ch] = rg[ch];
        }
    }
    for (int d = 0; d < 3; d++) {
        float r = 0.0f;
        for (uint32_t l = 0; l < max_level; l++)
            for (int ch = 0; ch < F; ch++) r += grad_feat[l * F + ch] * dydx[d][l * F + ch];
        dxyz[d] = r;
    }
}

/* ------------------------------------------------------------------ */
/* render backward: CR/backward.cu:445-2049 (modes 0/4/7/12/14; kernel 0) */
/* ------------------------------------------------------------------ */

typedef struct {
    int W, H;
    int C;                       /* channels of out_color                  */
    int level;                   /* 0: per-splat colours, >0: hash grid    */
    float beta;
    const uint32_t *ranges;      /* [tiles][2]                             */
    const uint32_t *point_list;
    const float *xy;             /* [P][2]                                 */
    const float *transmat;       /* [P][9]                                 */
    const float *normal_opacity; /* [P][4]                                 */
    const float *homotrans;      /* [P][16]                                */
    const float *ap_level;       /* [P]                                    */
    const float *colors;         /* [P][C] when level == 0                 */
    or_grid grid;
    const float *final_T;        /* [3][H][W] from the forward             */
    const uint32_t *n_contrib;   /* [2][H][W] from the forward             */
    const float *dL_dpix;        /* [C][H][W]                              */
    const float *dL_dothers;     /* [14][H][W]                             */
    /* accumulated outputs (zeroed by the caller) */
    float *dtable;               /* [rows][F]                              */
    float *dtransmat;            /* [P][9]                                 */
    float *dhomo;                /* [P][9]                                 */
    float *dmean2D;              /* [P][3]                                 */
    float *dnormal;              /* [P][3]                                 */
    float *dopacity;             /* [P]                                    */
    float *dcolors;              /* [P][C]; [P][hyb*F] in render mode 4,
                                    [P][total*F+1] in render mode 12        */
    float *gradsum;              /* [P]                                    */
    /* 0, 4 (hybrid_features, CR/backward.cu:987-1040) or 12 (adaptive_cat
     * training, :1425-1520) with `level` the packed (total << 16) | (active
     * grid levels << 8) | per-splat levels and colors the per-splat rows,
     * [P][hyb*F] in mode 4, [P][total*F+1] in mode 12, 14 (adaptive_zero
     * training, :1521-1590) with rows [P][hyb*F+1] */
    int render_mode;
    /* kernel_type 1-3 (CR/backward.cu:764-803, :1864-1909, :1963-2039) with
     * the per-splat shapes [P]; dshapes [P] accumulates dL/dshape */
    const float *shapes;
    int kernel_type;
    float *dshapes;
} or_render_bwd_args;

/* Grid levels the mode-4 backward differentiates (CR/backward.cu:576-612,
 * :993-999): the offsets are copied only up to the active count of bits 8-15
 * (the rest stay 0), and the levels are the largest i in 1..16 with
 * offsets[i] > offsets[i-1] over that copy.  The forward counts all of the
 * grid's levels, so with fewer active levels the backward recomputes and
 * differentiates only the active ones. */
static int cat_hash_levels_bwd(const or_grid *G, int active)
{
    int hl = 0;
    for (int i = 1; i < 17; i++) {
        int32_t a = (i - 1 <= active && i - 1 <= G->L) ? G->offsets[i - 1] : 0;
        int32_t b = (i <= active && i <= G->L) ? G->offsets[i] : 0;
        if (b > a) hl = i;
    }
    return hl;
}

static void render_pixel_bwd(const or_render_bwd_args *A, uint32_t tile, uint32_t px, uint32_t py, float *scr)
{
    const int W = A->W, H = A->H, C = A->C;
    const size_t HW = (size_t)W * (size_t)H;
    const size_t pid = (size_t)W * py + px;
    const float pxf = (float)px, pyf = (float)py;
    const uint32_t r0 = A->ranges[2 * tile], r1 = A->ranges[2 * tile + 1];
    const float *dO = A->dL_dothers;

    const float T_final = A->final_T[pid];
    float T = T_final;
    uint32_t contributor = r1 - r0;
    const uint32_t last_contributor = A->n_contrib[pid];
    const int median_contributor = (int)A->n_contrib[pid + HW];

    float *accum_rec = scr, *dL_dpixel = scr + C, *last_color = scr + 2 * C, *feat = scr + 3 * C,
          *grad_feat = scr + 4 * C;
    for (int c = 0; c < C; c++) {
        accum_rec[c] = 0.0f;
        last_color[c] = 0.0f;
        dL_dpixel[c] = A->dL_dpix[(size_t)c * HW + pid];
    }
    const float dL_ddepth = dO[0 * HW + pid];
    const float dL_daccum = dO[1 * HW + pid];
    const float dL_dreg = dO[6 * HW + pid];
    const float dL_dnormal2D[3] = {dO[2 * HW + pid], dO[3 * HW + pid], dO[4 * HW + pid]};
    const float dL_dmedian_depth = dO[5 * HW + pid];

    float last_depth = 0, last_normal[3] = {0, 0, 0};
    float accum_depth_rec = 0, accum_alpha_rec = 0, accum_normal_rec[3] = {0, 0, 0};
    const float final_D = A->final_T[pid + HW];
    const float final_D2 = A->final_T[pid + 2 * HW];
    const float final_A = 1 - T_final;
    float last_dL_dT = 0;
    float last_alpha = 0;

    for (uint32_t e = r1; e-- > r0;) {
        contributor--;
        if (contributor >= last_contributor) continue;
        const uint32_t id = A->point_list[e];
        const float *Tm = A->transmat + 9 * (size_t)id;
        const float Tu[3] = {Tm[0], Tm[1], Tm[2]}, Tv[3] = {Tm[3], Tm[4], Tm[5]}, Tw[3] = {Tm[6], Tm[7], Tm[8]};
        const float k[3] = {pxf * Tw[0] - Tu[0], pxf * Tw[1] - Tu[1], pxf * Tw[2] - Tu[2]};
        const float l[3] = {pyf * Tw[0] - Tv[0], pyf * Tw[1] - Tv[1], pyf * Tw[2] - Tv[2]};
        const float p[3] = {k[1] * l[2] - k[2] * l[1], k[2] * l[0] - k[0] * l[2], k[0] * l[1] - k[1] * l[0]};
        if (p[2] == 0.0f) continue;
        const float s[2] = {p[0] / p[2], p[1] / p[2]};
        const float rho3d = s[0] * s[0] + s[1] * s[1];
        const float d[2] = {A->xy[2 * id] - pxf, A->xy[2 * id + 1] - pyf};
        const float rho2d = 2.0f * (d[0] * d[0] + d[1] * d[1]);
        const float rho = fminf(rho3d, rho2d);
        const int use3d = rho3d <= rho2d;
        const float c_d = use3d ? (s[0] * Tw[0] + s[1] * Tw[1]) + Tw[2] : Tw[2];
        if (c_d < OR_NEAR) continue;
        const float *no = A->normal_opacity + 4 * (size_t)id;
        const float normal[3] = {no[0], no[1], no[2]};
        const float opa = no[3];

        float G, demon = 1.0f;
        /* kernel types: pf is the reference's dG_factor (2 dG/drho, but
         * dG/drho for the beta kernel), gs dG/dshape, gsc dG/dG_raw of a flex
         * splat (CR/backward.cu:764-803, :1963-1981) */
        float pf = 0.0f, gs = 0.0f, gsc = 1.0f, shp = 0.0f;
        const int kt = A->kernel_type;
        if (kt == 1) {
            if (rho >= 1.0f) continue;
            const float base = 1.0f - rho;
            shp = A->shapes[id];
            G = or_powf(base, shp);
            if (base > 1e-7f) {
                pf = -shp * G / base;
                gs = G * or_logf(base);
            }
        } else if (kt == 2) {
            const float power = -0.5f * rho;
            if (power > 0.0f) continue;
            const float g = or_expf(power);
            shp = A->shapes[id];
            G = g;
            pf = -g;
            if (shp > 0.0f) {
                demon = 1.0f + shp * g;
                G = (1.0f + shp) * g / demon;
                gsc = (1.0f + shp) / (demon * demon);
                gs = g * (1.0f - g) / (demon * demon);
            } else if (A->beta > 0.0f) {
                /* no per-splat beta: the settings' beta factor with demon = 1
                 * (CR/backward.cu:1875, :1910-1914) */
                gsc = (float)(1.0 + (double)A->beta);
            }
        } else if (kt == 3) {
            shp = A->shapes[id];
            const float rho_safe = fmaxf(rho, 1e-8f);
            const float pt = or_powf(rho_safe, 0.5f * shp);
            const float power = -0.5f * pt;
            if (power > 0.0f) continue;
            G = or_expf(power);
            pf = -0.5f * shp * G * pt / rho_safe;
            gs = -0.25f * G * pt * or_logf(rho_safe);
        } else {
            const float power = -0.5f * rho;
            if (power > 0.0f) continue;
            G = or_expf(power);
            if (A->beta > 0.0f) {
                demon = (float)(1.0 + (double)(A->beta * G));
                G = (float)((1.0 + (double)A->beta) * (double)G / (double)demon);
            }
        }
        const float alpha = fminf(0.99f, opa * G);
        if (alpha < 1.0f / 255.0f) continue;

        T = T / (1.f - alpha);
        const float dchannel_dcolor = alpha * T;
        float dL_dalpha = 0.0f;
        float dxyz[3] = {0.0f, 0.0f, 0.0f};
        const float *Hm = A->homotrans ? A->homotrans + 16 * (size_t)id : NULL;

        if (A->level == 0 && A->render_mode == 0) {
            for (int ch = 0; ch < C; ch++) {
                const float c = A->colors[(size_t)id * C + ch];
                accum_rec[ch] = last_alpha * last_color[ch] + (1.f - last_alpha) * accum_rec[ch];
                last_color[ch] = c;
                dL_dalpha += (c - accum_rec[ch]) * dL_dpixel[ch];
                A->dcolors[(size_t)id * C + ch] += dchannel_dcolor * dL_dpixel[ch];
            }
        } else {
            float xyz[3];
            if (use3d) {
                xyz[0] = s[0] * Hm[0] + s[1] * Hm[1] + Hm[3];
                xyz[1] = s[0] * Hm[4] + s[1] * Hm[5] + Hm[7];
                xyz[2] = s[0] * Hm[8] + s[1] * Hm[9] + Hm[11];
            } else {
                xyz[0] = Hm[3]; xyz[1] = Hm[7]; xyz[2] = Hm[11];
            }
            float sum_grad = 0.0f;
            for (int ch = 0; ch < C; ch++) {
                grad_feat[ch] = dchannel_dcolor * dL_dpixel[ch];
                sum_grad += fabsf(grad_feat[ch]);
            }
            A->gradsum[id] += sum_grad;
            const uint32_t ap = f2u_sat(floorf(A->ap_level[id]));
            if (A->render_mode == 4) {
                /* rows then the active grid levels (CR/backward.cu:987-1040) */
                const int pgd = (A->level & 0xFF) * A->grid.F;
                for (int ch = 0; ch < C; ch++) feat[ch] = 0.0f;
                for (int i = 0; i < pgd; i++) feat[i] = A->colors[(size_t)id * pgd + i];
                const int hl = cat_hash_levels_bwd(&A->grid, (A->level >> 8) & 0xFF);
                if (hl > 0) {
                    or_grid G = A->grid;
                    G.L = hl;
                    qf_backward(&G, xyz, ap, C - pgd, grad_feat + pgd, feat + pgd, A->dtable, dxyz);
                }
                for (int i = 0; i < pgd; i++) A->dcolors[(size_t)id * pgd + i] += grad_feat[i];
            } else if (A->render_mode == 7) {
                /* adaptive_add (CR/backward.cu:1108-1189): rows [total*F |
                 * weight]; each channel passes weight * g to the row and
                 * (1 - weight) * g to the grid (hl levels); the weight's slot
                 * receives sum (row - grid) . g times weight * (1 - weight), the
                 * gradient of the logit the weight is a sigmoid of.  The blend
                 * terms use the forward's features. */
                const int total = (A->level >> 16) & 0xFF, hl = (A->level >> 8) & 0xFF;
                const int F = A->grid.F, tdim = total * F;
                const float *gf = A->colors + (size_t)id * (size_t)(tdim + 1);
                float *dc = A->dcolors + (size_t)id * (size_t)(tdim + 1);
                const float wt = gf[tdim], iw = 1.0f - wt;
                float hf[64], gh[64];
                for (int i = 0; i < 64; i++) hf[i] = 0.0f;
                if (hl > 0) {
                    or_grid G = A->grid;
                    G.L = hl;
                    for (int i = 0; i < hl * F; i++) gh[i] = iw * grad_feat[i];
                    qf_backward(&G, xyz, ap, hl * F, gh, hf, A->dtable, dxyz);
                }
                for (int ch = 0; ch < C; ch++) feat[ch] = 0.0f;
                float dweight = 0.0f;
                for (int i = 0; i < tdim; i++) {
                    dc[i] += wt * grad_feat[i];
                    dweight += grad_feat[i] * (gf[i] - hf[i]);
                    feat[i] = fmaf(wt, gf[i], iw * hf[i]);
                }
                dc[tdim] += dweight * wt * iw;
            } else if (A->render_mode == 14) {
                /* adaptive_zero training (CR/backward.cu:1521-1590): rows
                 * [hyb*F | weight]; the coarse channels pass their gradient to
                 * the row; when the weight is > 1e-6 the hl grid levels pass
                 * weight * g to the table and grid . g to the weight.  The
                 * blend terms use the forward's features, as in mode 12. */
                const int hl = (A->level >> 8) & 0xFF, hyb = A->level & 0xFF;
                const int F = A->grid.F, pgd = hyb * F;
                const float *gf = A->colors + (size_t)id * (size_t)(pgd + 1);
                float *dc = A->dcolors + (size_t)id * (size_t)(pgd + 1);
                const float wt = gf[pgd];
                for (int ch = 0; ch < C; ch++) feat[ch] = 0.0f;
                for (int i = 0; i < pgd; i++) {
                    feat[i] = gf[i];
                    dc[i] += grad_feat[i];
                }
                float dweight = 0.0f;
                if (hl > 0 && wt > 1e-6f) {
                    or_grid G = A->grid;
                    G.L = hl;
                    float hf[64], gh[64];
                    for (int i = 0; i < hl * F; i++) gh[i] = wt * grad_feat[pgd + i];
                    qf_backward(&G, xyz, ap, hl * F, gh, hf, A->dtable, dxyz);
                    for (int i = 0; i < hl * F; i++) {
                        dweight += hf[i] * grad_feat[pgd + i];
                        feat[pgd + i] = wt * hf[i];
                    }
                }
                dc[pgd] += dweight;
            } else if (A->render_mode == 12) {
                /* adaptive_cat training (CR/backward.cu:1425-1520): rows
                 * [total*F | weight]; the coarse hyb*F channels pass their
                 * gradient to the row, the hl grid levels split theirs into
                 * weight * g for the row, (1 - weight) * g for the table and
                 * (row - grid) . g for the weight.  The blend terms of dL/dalpha
                 * use the forward's features (the reference reads an array it
                 * never wrote here). */
                const int total = (A->level >> 16) & 0xFF, hl = (A->level >> 8) & 0xFF, hyb = A->level & 0xFF;
                const int F = A->grid.F, tdim = total * F, fs = hyb * F;
                const float *gf = A->colors + (size_t)id * (size_t)(tdim + 1);
                float *dc = A->dcolors + (size_t)id * (size_t)(tdim + 1);
                const float wt = gf[tdim];
                for (int ch = 0; ch < C; ch++) feat[ch] = 0.0f;
                for (int i = 0; i < fs; i++) {
                    feat[i] = gf[i];
                    dc[i] += grad_feat[i];
                }
                float dweight = 0.0f;
                if (hl > 0) {
                    or_grid G = A->grid;
                    G.L = hl;
                    float hf[64], gh[64];
                    for (int i = 0; i < hl * F; i++) gh[i] = (1.0f - wt) * grad_feat[fs + i];
                    qf_backward(&G, xyz, ap, hl * F, gh, hf, A->dtable, dxyz);
                    for (int i = 0; i < hl * F; i++) {
                        dc[fs + i] += wt * grad_feat[fs + i];
                        dweight += (gf[fs + i] - hf[i]) * grad_feat[fs + i];
                        feat[fs + i] = fmaf(wt, gf[fs + i], (1.0f - wt) * hf[i]);
                    }
                }
                dc[tdim] += dweight;
            } else {
                qf_backward(&A->grid, xyz, ap, C, grad_feat, feat, A->dtable, dxyz);
            }
            for (int ch = 0; ch < C; ch++) {
                const float c = feat[ch];
                accum_rec[ch] = last_alpha * last_color[ch] + (1.f - last_alpha) * accum_rec[ch];
                last_color[ch] = c;
                dL_dalpha += (c - accum_rec[ch]) * dL_dpixel[ch];
            }
        }

        /* RENDER_AXUTILITY terms: backward.cu:1815-1855 */
        float dL_dz = 0.0f, dL_dweight = 0.0f;
        const float m_d = OR_FAR / (OR_FAR - OR_NEAR) * (1 - OR_NEAR / c_d);
        const float dmd_dd = (OR_FAR * OR_NEAR) / ((OR_FAR - OR_NEAR) * c_d * c_d);
        if ((int)contributor == median_contributor - 1) dL_dz += dL_dmedian_depth;
        dL_dweight += (final_D2 + m_d * m_d * final_A - 2 * m_d * final_D) * dL_dreg;
        dL_dalpha += dL_dweight - last_dL_dT;
        last_dL_dT = dL_dweight * alpha + (1 - alpha) * last_dL_dT;
        const float dL_dmd = 2.0f * (T * alpha) * (m_d * final_A - final_D) * dL_dreg;
        dL_dz += dL_dmd * dmd_dd;
        accum_depth_rec = last_alpha * last_depth + (1.f - last_alpha) * accum_depth_rec;
        last_depth = c_d;
        dL_dalpha += (c_d - accum_depth_rec) * dL_ddepth;
        accum_alpha_rec = last_alpha * 1.0f + (1.f - last_alpha) * accum_alpha_rec;
        dL_dalpha += (1 - accum_alpha_rec) * dL_daccum;
        for (int ch = 0; ch < 3; ch++) {
            accum_normal_rec[ch] = last_alpha * last_normal[ch] + (1.f - last_alpha) * accum_normal_rec[ch];
            last_normal[ch] = normal[ch];
            dL_dalpha += (normal[ch] - accum_normal_rec[ch]) * dL_dnormal2D[ch];
            A->dnormal[3 * (size_t)id + ch] += alpha * T * dL_dnormal2D[ch];
        }
        dL_dalpha *= T;
        last_alpha = alpha;

        float dL_dG = opa * dL_dalpha;
        if (kt != 0) {
            A->dshapes[id] += dL_dalpha * opa * gs;
            if (kt == 2) dL_dG *= gsc;
        } else if (A->beta > 0.0f) {
            const float dG_dg = (float)((1.0 + (double)A->beta) / (double)(demon * demon));
            dL_dG *= dG_dg;
        }
        dL_dz += alpha * T * dL_ddepth;

        /* homotrans gradient (backward.cu:1921-1952) */
        float dL_duv[2] = {0.0f, 0.0f};
        if (Hm && A->level > 0) {
            if (use3d) {
                dL_duv[0] = dxyz[0] * Hm[0] + dxyz[1] * Hm[4] + dxyz[2] * Hm[8];
                dL_duv[1] = dxyz[0] * Hm[1] + dxyz[1] * Hm[5] + dxyz[2] * Hm[9];
                float *h = A->dhomo + 9 * (size_t)id;
                h[0] += dxyz[0] * s[0]; h[1] += dxyz[1] * s[0]; h[2] += dxyz[2] * s[0];
                h[3] += dxyz[0] * s[1]; h[4] += dxyz[1] * s[1]; h[5] += dxyz[2] * s[1];
            }
            float *h = A->dhomo + 9 * (size_t)id;
            h[6] += dxyz[0]; h[7] += dxyz[1]; h[8] += dxyz[2];
        }

        if (use3d) {
            /* backward.cu:1956-2011 with dG_factor = -G (kernel types: pf) */
            const float dG_factor = kt ? pf : -G;
            float dL_ds[2] = {dL_dG * dG_factor * s[0] + dL_dz * Tw[0], dL_dG * dG_factor * s[1] + dL_dz * Tw[1]};
            dL_ds[0] += dL_duv[0];
            dL_ds[1] += dL_duv[1];
            const float dz_dTw[3] = {s[0], s[1], 1.0f};
            const float dsx_pz = dL_ds[0] / p[2], dsy_pz = dL_ds[1] / p[2];
            const float dL_dp[3] = {dsx_pz, dsy_pz, -(dsx_pz * s[0] + dsy_pz * s[1])};
            /* dL_dk = cross(l, dL_dp), dL_dl = cross(dL_dp, k) */
            const float dk[3] = {l[1] * dL_dp[2] - l[2] * dL_dp[1], l[2] * dL_dp[0] - l[0] * dL_dp[2],
                                 l[0] * dL_dp[1] - l[1] * dL_dp[0]};
            const float dl[3] = {dL_dp[1] * k[2] - dL_dp[2] * k[1], dL_dp[2] * k[0] - dL_dp[0] * k[2],
                                 dL_dp[0] * k[1] - dL_dp[1] * k[0]};
            float *t = A->dtransmat + 9 * (size_t)id;
            for (int r = 0; r < 3; r++) {
                t[r] += -dk[r];
                t[3 + r] += -dl[r];
                t[6 + r] += pxf * dk[r] + pyf * dl[r] + dL_dz * dz_dTw[r];
            }
        } else {
            const float dG_factor_2d = kt ? pf * 2.0f : -G * 2.0f;
            const float dG_ddelx = dG_factor_2d * d[0], dG_ddely = dG_factor_2d * d[1];
            A->dmean2D[3 * (size_t)id + 0] += dL_dG * dG_ddelx;
            A->dmean2D[3 * (size_t)id + 1] += dL_dG * dG_ddely;
            A->dtransmat[9 * (size_t)id + 8] += dL_dz;
        }
        A->dopacity[id] += G * dL_dalpha;
    }
}

/* Backward of the render for every pixel, tiles in order, pixels row-major
 * inside a tile (the accumulation order of every per-splat sum). */
void or_render_backward(const or_render_bwd_args *A)
{
    const int gx = (A->W + OR_BLOCK - 1) / OR_BLOCK, gy = (A->H + OR_BLOCK - 1) / OR_BLOCK;
    float *scr = (float *)malloc(sizeof(float) * 5 * (size_t)(A->C > 0 ? A->C : 1));
    for (int ty = 0; ty < gy; ty++)
        for (int tx = 0; tx < gx; tx++)
            for (int yy = 0; yy < OR_BLOCK; yy++)
                for (int xx = 0; xx < OR_BLOCK; xx++) {
                    uint32_t px = (uint32_t)(tx * OR_BLOCK + xx), py = (uint32_t)(ty * OR_BLOCK + yy);
                    if (px >= (uint32_t)A->W || py >= (uint32_t)A->H) continue;
                    render_pixel_bwd(A, (uint32_t)(ty * gx + tx), px, py, scr);
                }
    free(scr);
}

/* ------------------------------------------------------------------ */
/* preprocess backward: CR/backward.cu:2056-2274, :20-140               */
/* ------------------------------------------------------------------ */

/* computeColorFromSH backward (CR/backward.cu:20-140): dL/dsh of splat idx
 * and the view-direction term added to dmeans[idx]. */
static void sh_backward(int idx, int deg, int M, const float *means, const float *campos, const float *shs,
                        const uint8_t *clamped, const float *dcolor, float *dmeans, float *dshs)
{
    const float C0 = 0.28209479177387814f, C1 = 0.4886025119029199f;
    const float C2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f, -1.0925484305920792f,
                         0.5462742152960396f};
    const float C3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f, 0.3731763325901154f,
                         -0.4570457994644658f, 1.445305721320277f, -0.5900435899266435f};
    const float *pos = means + 3 * (size_t)idx;
    const float dir_orig[3] = {pos[0] - campos[0], pos[1] - campos[1], pos[2] - campos[2]};
    const float len = sqrtf(dir_orig[0] * dir_orig[0] + dir_orig[1] * dir_orig[1] + dir_orig[2] * dir_orig[2]);
    const float x = dir_orig[0] / len, y = dir_orig[1] / len, z = dir_orig[2] / len;
    const float *sh = shs + (size_t)idx * M * 3;
    float g[3];
    for (int c = 0; c < 3; c++) g[c] = dcolor[3 * (size_t)idx + c] * (clamped[3 * (size_t)idx + c] ? 0.0f : 1.0f);
    float *dsh = dshs + (size_t)idx * M * 3;
    float dx[3] = {0, 0, 0}, dy[3] = {0, 0, 0}, dz[3] = {0, 0, 0};
#define SH(i, c) sh[3 * (i) + (c)]
#define DSH(i, v) for (int c = 0; c < 3; c++) dsh[3 * (i) + c] = (v) * g[c]
    DSH(0, C0);
    if (deg > 0) {
        DSH(1, -C1 * y); DSH(2, C1 * z); DSH(3, -C1 * x);
        for (int c = 0; c < 3; c++) { dx[c] = -C1 * SH(3, c); dy[c] = -C1 * SH(1, c); dz[c] = C1 * SH(2, c); }
        if (deg > 1) {
            const float xx = x * x, yy = y * y, zz = z * z, xy = x * y, yz = y * z, xz = x * z;
            DSH(4, C2[0] * xy); DSH(5, C2[1] * yz); DSH(6, C2[2] * (2.f * zz - xx - yy));
            DSH(7, C2[3] * xz); DSH(8, C2[4] * (xx - yy));
            for (int c = 0; c < 3; c++) {
                dx[c] += C2[0] * y * SH(4, c) + C2[2] * 2.f * -x * SH(6, c) + C2[3] * z * SH(7, c) + C2[4] * 2.f * x * SH(8, c);
                dy[c] += C2[0] * x * SH(4, c) + C2[1] * z * SH(5, c) + C2[2] * 2.f * -y * SH(6, c) + C2[4] * 2.f * -y * SH(8, c);
                dz[c] += C2[1] * y * SH(5, c) + C2[2] * 2.f * 2.f * z * SH(6, c) + C2[3] * x * SH(7, c);
            }
            if (deg > 2) {
                DSH(9, C3[0] * y * (3.f * xx - yy)); DSH(10, C3[1] * xy * z); DSH(11, C3[2] * y * (4.f * zz - xx - yy));
                DSH(12, C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy)); DSH(13, C3[4] * x * (4.f * zz - xx - yy));
                DSH(14, C3[5] * z * (xx - yy)); DSH(15, C3[6] * x * (xx - 3.f * yy));
                for (int c = 0; c < 3; c++) {
                    dx[c] += (C3[0] * SH(9, c) * 3.f * 2.f * xy + C3[1] * SH(10, c) * yz + C3[2] * SH(11, c) * -2.f * xy +
                              C3[3] * SH(12, c) * -3.f * 2.f * xz + C3[4] * SH(13, c) * (-3.f * xx + 4.f * zz - yy) +
                              C3[5] * SH(14, c) * 2.f * xz + C3[6] * SH(15, c) * 3.f * (xx - yy));
                    dy[c] += (C3[0] * SH(9, c) * 3.f * (xx - yy) + C3[1] * SH(10, c) * xz +
                              C3[2] * SH(11, c) * (-3.f * yy + 4.f * zz - xx) + C3[3] * SH(12, c) * -3.f * 2.f * yz +
                              C3[4] * SH(13, c) * -2.f * xy + C3[5] * SH(14, c) * -2.f * yz +
                              C3[6] * SH(15, c) * -3.f * 2.f * xy);
                    dz[c] += (C3[1] * SH(10, c) * xy + C3[2] * SH(11, c) * 4.f * 2.f * yz +
                              C3[3] * SH(12, c) * 3.f * (2.f * zz - xx - yy) + C3[4] * SH(13, c) * 4.f * 2.f * xz +
                              C3[5] * SH(14, c) * (xx - yy));
                }
            }
        }
    }
#undef SH
#undef DSH
    /* dL/ddir = (dRGBdx . dL_dRGB, ...), then dnormvdv (auxiliary.h:133-143) */
    const float ddir[3] = {dx[0] * g[0] + dx[1] * g[1] + dx[2] * g[2], dy[0] * g[0] + dy[1] * g[1] + dy[2] * g[2],
                           dz[0] * g[0] + dz[1] * g[1] + dz[2] * g[2]};
    const float *v = dir_orig;
    const float sum2 = v[0] * v[0] + v[1] * v[1] + v[2] * v[2];
    const float invsum32 = 1.0f / sqrtf(sum2 * sum2 * sum2);
    dmeans[3 * (size_t)idx + 0] += ((+sum2 - v[0] * v[0]) * ddir[0] - v[1] * v[0] * ddir[1] - v[2] * v[0] * ddir[2]) * invsum32;
    dmeans[3 * (size_t)idx + 1] += (-v[0] * v[1] * ddir[0] + (sum2 - v[1] * v[1]) * ddir[1] - v[2] * v[1] * ddir[2]) * invsum32;
    dmeans[3 * (size_t)idx + 2] += (-v[0] * v[2] * ddir[0] - v[1] * v[2] * ddir[1] + (sum2 - v[2] * v[2]) * ddir[2]) * invsum32;
}

/* preprocessCUDA backward (CR/backward.cu:2216-2274) for every splat with
 * radii > 0: compute_transmat_aabb (:2056-2214) folds the render's dL/dmean2D
 * into dL/dT, maps dL/dT and dL/dhomotrans (the same splat2world matrix M)
 * to means, scales and rotations, differentiates the normalised, view-facing
 * normal, adds the SH term, then overwrites dmean2D with the densification
 * statistic dL/dTu.z * depth * W/2, dL/dTv.z * depth * H/2 of the render's
 * dL/dT (the fold changes a local copy only, as the reference's glm
 * dL_dT).  dmeans, dscales, drots are assigned (dmeans then gets the SH term
 * added). */
void or_preprocess_backward(int P, const float *means, const float *scales, const float *rots, const int32_t *radii,
                            const float *transmat, const float *view, const float *proj, int W, int H,
                            const float *shs, int sh_degree, int sh_coeffs, const float *campos, const uint8_t *clamped,
                            const float *dcolors, const float *dtransmat, const float *dhomo, const float *dnormal,
                            float *dmean2D, float *dmeans, float *dscales, float *drots, float *dshs)
{
    for (int idx = 0; idx < P; idx++) {
        if (!(radii[idx] > 0)) continue;
        const float *po = means + 3 * (size_t)idx;
        /* quat_to_rotmat (auxiliary.h:218-240), glm column-major R[col][row] */
        const float *q = rots + 4 * (size_t)idx;
        const float sq = 1.0f / sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
        const float qw = q[0] * sq, qx = q[1] * sq, qy = q[2] * sq, qz = q[3] * sq;
        float R[3][3];
        R[0][0] = 1.f - 2.f * (qy * qy + qz * qz); R[0][1] = 2.f * (qx * qy + qw * qz); R[0][2] = 2.f * (qx * qz - qw * qy);
        R[1][0] = 2.f * (qx * qy - qw * qz); R[1][1] = 1.f - 2.f * (qx * qx + qz * qz); R[1][2] = 2.f * (qy * qz + qw * qx);
        R[2][0] = 2.f * (qx * qz + qw * qy); R[2][1] = 2.f * (qy * qz - qw * qx); R[2][2] = 1.f - 2.f * (qx * qx + qy * qy);
        const float sc[2] = {scales[2 * (size_t)idx], scales[2 * (size_t)idx + 1]};
        /* L = R * scale_to_mat(scale, 1.0f): columns R0*sx, R1*sy, R2 */
        float Lc[3][3];
        for (int r = 0; r < 3; r++) { Lc[0][r] = R[0][r] * (1.0f * sc[0]); Lc[1][r] = R[1][r] * (1.0f * sc[1]); Lc[2][r] = R[2][r]; }
        /* M = mat3x4((L0,0), (L1,0), (p,1)); world2ndc[col][row] = proj[4*row+col];
         * ndc2pix columns (W/2,0,0,(W-1)/2), (0,H/2,0,(H-1)/2), (0,0,0,1) */
        const float M[3][4] = {{Lc[0][0], Lc[0][1], Lc[0][2], 0.0f}, {Lc[1][0], Lc[1][1], Lc[1][2], 0.0f},
                               {po[0], po[1], po[2], 1.0f}};
        const float N[3][4] = {{(float)W / 2.0f, 0.0f, 0.0f, (float)(W - 1) / 2.0f},
                               {0.0f, (float)H / 2.0f, 0.0f, (float)(H - 1) / 2.0f}, {0.0f, 0.0f, 0.0f, 1.0f}};
        /* P = world2ndc * ndc2pix: column c, row r = sum_k world2ndc[k][r] * N[c][k] */
        float Pm[3][4];
        for (int c = 0; c < 3; c++)
            for (int r = 0; r < 4; r++) {
                float acc = proj[4 * r + 0] * N[c][0];
                acc = acc + proj[4 * r + 1] * N[c][1];
                acc = acc + proj[4 * r + 2] * N[c][2];
                acc = acc + proj[4 * r + 3] * N[c][3];
                Pm[c][r] = acc;
            }
        /* T = transpose(M) * P: T[c][i] = dot(M[i], P[c]) (glm column c, row i) */
        float Tt[3][3];
        for (int c = 0; c < 3; c++)
            for (int i = 0; i < 3; i++) {
                float acc = M[i][0] * Pm[c][0];
                acc = acc + M[i][1] * Pm[c][1];
                acc = acc + M[i][2] * Pm[c][2];
                acc = acc + M[i][3] * Pm[c][3];
                Tt[c][i] = acc;
            }
        /* normal = transformVec4x3(L2, view) (auxiliary.h:104-112) */
        const float nrm[3] = {view[0] * Lc[2][0] + view[4] * Lc[2][1] + view[8] * Lc[2][2],
                              view[1] * Lc[2][0] + view[5] * Lc[2][1] + view[9] * Lc[2][2],
                              view[2] * Lc[2][0] + view[6] * Lc[2][1] + view[10] * Lc[2][2]};

        const float *dTm = dtransmat + 9 * (size_t)idx;
        float dT[9]; /* glm columns dT[0..2], dT[3..5], dT[6..8] */
        for (int r = 0; r < 9; r++) dT[r] = dTm[r];
        float *dm2 = dmean2D + 3 * (size_t)idx;
        if (dm2[0] != 0 || dm2[1] != 0) {
            const float tv[3] = {9.0f, 9.0f, -1.0f};
            const float T2sq[3] = {Tt[2][0] * Tt[2][0], Tt[2][1] * Tt[2][1], Tt[2][2] * Tt[2][2]};
            const float dd = tv[0] * T2sq[0] + tv[1] * T2sq[1] + tv[2] * T2sq[2];
            const float inv = 1.0f / dd;
            const float f[3] = {tv[0] * inv, tv[1] * inv, tv[2] * inv};
            float dT0[3], dT1[3], dT3[3], df[3];
            for (int r = 0; r < 3; r++) {
                dT0[r] = dm2[0] * f[r] * Tt[2][r];
                dT1[r] = dm2[1] * f[r] * Tt[2][r];
                dT3[r] = dm2[0] * f[r] * Tt[0][r] + dm2[1] * f[r] * Tt[1][r];
                df[r] = dm2[0] * Tt[0][r] * Tt[2][r] + dm2[1] * Tt[1][r] * Tt[2][r];
            }
            const float dL_dd = (float)((double)(df[0] * f[0] + df[1] * f[1] + df[2] * f[2]) * (-1.0 / (double)dd));
            for (int r = 0; r < 3; r++) {
                const float ddT3 = tv[r] * Tt[2][r] * 2.0f;
                dT3[r] += dL_dd * ddT3;
                dT[r] += dT0[r];
                dT[3 + r] += dT1[r];
                dT[6 + r] += dT3[r];
            }
        }
        /* dL_dM = P * transpose(dL_dT) + dL_dhomo: column i, row r =
         * sum_c P[c][r] * dT[3c + i] */
        const float *hh = dhomo + 9 * (size_t)idx;
        float dM[3][4];
        for (int i = 0; i < 3; i++)
            for (int r = 0; r < 4; r++) {
                float acc = Pm[0][r] * dT[0 + i];
                acc = acc + Pm[1][r] * dT[3 + i];
                acc = acc + Pm[2][r] * dT[6 + i];
                dM[i][r] = acc + (r < 3 ? hh[3 * i + r] : 0.0f);
            }
        /* normal normalisation backward (backward.cu:2151-2168) */
        const float *gn = dnormal + 3 * (size_t)idx;
        const float nlen = sqrtf(nrm[0] * nrm[0] + nrm[1] * nrm[1] + nrm[2] * nrm[2]);
        float gu[3] = {0.0f, 0.0f, 0.0f};
        if (nlen > 1e-7f) {
            const float dot = gn[0] * nrm[0] + gn[1] * nrm[1] + gn[2] * nrm[2];
            for (int r = 0; r < 3; r++) gu[r] = (gn[r] - dot * nrm[r] / nlen) / nlen;
        }
        /* transformVec4x3Transpose (auxiliary.h:115-123) */
        float dtn[3] = {view[0] * gu[0] + view[1] * gu[1] + view[2] * gu[2],
                        view[4] * gu[0] + view[5] * gu[1] + view[6] * gu[2],
                        view[8] * gu[0] + view[9] * gu[1] + view[10] * gu[2]};
        /* DUAL_VISIABLE (backward.cu:2172-2177) */
        const float pv[3] = {view[0] * po[0] + view[4] * po[1] + view[8] * po[2] + view[12],
                             view[1] * po[0] + view[5] * po[1] + view[9] * po[2] + view[13],
                             view[2] * po[0] + view[6] * po[1] + view[10] * po[2] + view[14]};
        const float cosv = -(pv[0] * nrm[0] + pv[1] * nrm[1] + pv[2] * nrm[2]);
        const float mul = cosv > 0 ? 1.0f : -1.0f;
        for (int r = 0; r < 3; r++) dtn[r] = mul * dtn[r];
        /* dL_dRS columns dM[0].xyz, dM[1].xyz, dtn; dL_dR = (dRS0*sx, dRS1*sy, dRS2) */
        float dR[3][3];
        for (int r = 0; r < 3; r++) { dR[0][r] = dM[0][r] * sc[0]; dR[1][r] = dM[1][r] * sc[1]; dR[2][r] = dtn[r]; }
        /* quat_to_rotmat_vjp (auxiliary.h:244-288); v_R[col][row] */
        float *dq = drots + 4 * (size_t)idx;
        dq[0] = 2.f * (qx * (dR[1][2] - dR[2][1]) + qy * (dR[2][0] - dR[0][2]) + qz * (dR[0][1] - dR[1][0]));
        dq[1] = 2.f * (-2.f * qx * (dR[1][1] + dR[2][2]) + qy * (dR[0][1] + dR[1][0]) + qz * (dR[0][2] + dR[2][0]) +
                       qw * (dR[1][2] - dR[2][1]));
        dq[2] = 2.f * (qx * (dR[0][1] + dR[1][0]) - 2.f * qy * (dR[0][0] + dR[2][2]) + qz * (dR[1][2] + dR[2][1]) +
                       qw * (dR[2][0] - dR[0][2]));
        dq[3] = 2.f * (qx * (dR[0][2] + dR[2][0]) + qy * (dR[1][2] + dR[2][1]) - 2.f * qz * (dR[0][0] + dR[1][1]) +
                       qw * (dR[0][1] - dR[1][0]));
        dscales[2 * (size_t)idx + 0] = dM[0][0] * R[0][0] + dM[0][1] * R[0][1] + dM[0][2] * R[0][2];
        dscales[2 * (size_t)idx + 1] = dM[1][0] * R[1][0] + dM[1][1] * R[1][1] + dM[1][2] * R[1][2];
        dmeans[3 * (size_t)idx + 0] = dM[2][0];
        dmeans[3 * (size_t)idx + 1] = dM[2][1];
        dmeans[3 * (size_t)idx + 2] = dM[2][2];

        if (shs) sh_backward(idx, sh_degree, sh_coeffs, means, campos, shs, clamped, dcolors, dmeans, dshs);

        /* densification statistic (backward.cu:2268-2271) */
        const float depth = transmat[9 * (size_t)idx + 8];
        const int Wi = W, Hi = H;
        dm2[0] = (float)((double)(dTm[2] * depth) * 0.5 * (double)(float)Wi);
        dm2[1] = (float)((double)(dTm[5] * depth) * 0.5 * (double)(float)Hi);
    }
}

/* ------------------------------------------------------------------ */
/* GridEncoder backward: GE/src/gridencoder.cu:196-242, :245-366        */
/* ------------------------------------------------------------------ */

/* grad_table[entry] += w * grad[b][l*F + ch] over every corner (binary32
 * tables), and, when grad_inputs is given, grad_inputs[b][d] =
 * sum_l sum_ch grad[b][l*F+ch] * dy_dx[b][l][d][ch] with the forward's dy_dx
 * (w starts at scale, not scale * grad_scale).  Out-of-range inputs get no
 * table gradient and zero input gradient. */
void or_grid_encode_backward(const or_grid *G, int B, const float *inputs, const float *grad, float *grad_table,
                             float *grad_inputs)
{
    const int L = G->L, F = G->F;
    for (int b = 0; b < B; b++) {
        const float *u = inputs + 3 * (size_t)b;
        const int oob = (u[0] < 0 || u[0] > 1 || u[1] < 0 || u[1] > 1 || u[2] < 0 || u[2] > 1);
        if (grad_inputs) grad_inputs[3 * (size_t)b] = grad_inputs[3 * (size_t)b + 1] = grad_inputs[3 * (size_t)b + 2] = 0.0f;
        if (oob) continue;
        float gi[3] = {0.0f, 0.0f, 0.0f};
        for (int l = 0; l < L; l++) {
            uint32_t hsize = (uint32_t)(G->offsets[l + 1] - G->offsets[l]);
            float scale; uint32_t res;
            or_level_scale(G->S, G->H, l, &scale, &res);
            size_t base = (size_t)(uint32_t)G->offsets[l] * (size_t)F;
            const float *gr = grad + (size_t)b * L * F + (size_t)l * F;
            float pos[3], der[3]; uint32_t g[3];
            for (int d = 0; d < 3; d++) {
                pos[d] = u[d] * scale + (G->align_corners ? 0.0f : 0.5f);
                g[d] = f2u_sat(floorf(pos[d]));
                pos[d] = pos[d] - (float)g[d];
                if (G->interp == 1) { der[d] = 6.0f * pos[d] * (1.0f - pos[d]); pos[d] = pos[d] * pos[d] * (3.0f - 2.0f * pos[d]); }
                else der[d] = 1.0f;
            }
            for (uint32_t corner = 0; corner < 8; corner++) {
                float w = 1.0f; uint32_t q[3];
                for (int d = 0; d < 3; d++) {
                    if ((corner & (1u << d)) == 0) { w *= 1 - pos[d]; q[d] = g[d]; }
                    else { w *= pos[d]; q[d] = g[d] + 1u; }
                }
                size_t e = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
                for (int ch = 0; ch < F; ch++) grad_table[e + ch] += w * gr[ch];
            }
            if (!grad_inputs) continue;
            for (int gd = 0; gd < 3; gd++) {
                float rg[16];
                for (int ch = 0; ch < F; ch++) rg[ch] = 0.0f;
                for (uint32_t idx = 0; idx < 4; idx++) {
                    float w = scale; uint32_t q[3];
                    for (int nd = 0; nd < 2; nd++) {
                        const int d = (nd >= gd) ? nd + 1 : nd;
                        if ((idx & (1u << nd)) == 0) { w *= 1 - pos[d]; q[d] = g[d]; }
                        else { w *= pos[d]; q[d] = g[d] + 1u; }
                    }
                    q[gd] = g[gd];
                    size_t el = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
                    q[gd] = g[gd] + 1u;
                    size_t er = base + (size_t)grid_index(G->align_corners, hsize, res, q) * F;
                    for (int ch = 0; ch < F; ch++) rg[ch] += w * (table_at(G, er + ch) - table_at(G, el + ch)) * der[gd];
                }
                for (int ch = 0; ch < F; ch++) gi[gd] += gr[ch] * rg[ch];
            }
        }
        if (grad_inputs) for (int d = 0; d < 3; d++) grad_inputs[3 * (size_t)b + d] = gi[d];
    }
}
