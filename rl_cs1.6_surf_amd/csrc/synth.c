/* synth.c — analytic unsigned distance grids for synthetic surf scenes.
 *
 * Builds the [nz][ny][nx] f32 grid the renderer consumes, with the
 * reference's grid contract (python/surfgym/vision.py grid_dims :310-322):
 * voxel (ix,iy,iz) is sampled at mins + (i + 0.5)*cell (src/env.c:680-682)
 * and holds the Euclidean distance from that point to the nearest solid, 0
 * inside a solid — the convention of the reference's EDT bake
 * (vision.py:428-432), evaluated exactly instead of from an occupancy grid,
 * like the analytic fixtures of the reference's own renderer tests
 * (tests/python/test_pinhole.py:186-202, test_surfmask.py:177-193).
 *
 * Solids: an optional ground half-space z <= ground_z, surf ramps
 * (triangular prisms: a symmetric triangle of half-base b and height h in
 * the vertical plane across the ramp, extruded along a horizontal axis) and
 * boxes rotated about z. Values are min(distance, trunc).
 *
 * Exact per voxel; the speed comes from culling per 8x8x8 block: with c the
 * block centre and R its half-diagonal, every voxel v of the block has
 * dist(v) <= dist(c) + R =: ub, and a solid whose bounding box lies farther
 * than ub from the block cannot be nearest to any of its voxels.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <stddef.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define SYNTH_API __attribute__((visibility("default")))

typedef struct SynthPrism {
    float cx, cy, z0;      /* centre of the base line, base height */
    float ax, ay;          /* unit horizontal axis the ramp runs along */
    float half_len;        /* half length along the axis */
    float half_base;       /* b: half width of the base */
    float height;          /* h: apex height above the base */
} SynthPrism;

typedef struct SynthBox {
    float cx, cy, cz;      /* centre */
    float hx, hy, hz;      /* half extents in the box frame */
    float cos_a, sin_a;    /* rotation about z */
} SynthBox;

typedef struct Aabb { double lo[3], hi[3]; } Aabb;

static double seg_dist2(double px, double py, double ax, double ay, double bx, double by) {
    const double ex = bx - ax, ey = by - ay;
    const double wx = px - ax, wy = py - ay;
    double t = (wx * ex + wy * ey) / (ex * ex + ey * ey);
    if (t < 0.0) t = 0.0;
    if (t > 1.0) t = 1.0;
    const double dx = wx - t * ex, dy = wy - t * ey;
    return dx * dx + dy * dy;
}

static double prism_dist(const SynthPrism* s, double x, double y, double z) {
    const double rx = x - s->cx, ry = y - s->cy;
    const double along = rx * s->ax + ry * s->ay;
    const double across = fabs(-rx * s->ay + ry * s->ax);
    const double w = z - s->z0;
    const double b = s->half_base, h = s->height;
    double dl = fabs(along) - s->half_len;
    if (dl < 0.0) dl = 0.0;
    double dt2;
    if (w >= 0.0 && across <= b && w <= h * (1.0 - across / b)) {
        dt2 = 0.0;
    } else {
        const double d1 = seg_dist2(across, w, 0.0, 0.0, b, 0.0);   /* base */
        const double d2 = seg_dist2(across, w, b, 0.0, 0.0, h);     /* slanted face */
        dt2 = d1 < d2 ? d1 : d2;
    }
    return sqrt(dt2 + dl * dl);
}

static double box_dist(const SynthBox* s, double x, double y, double z) {
    const double rx = x - s->cx, ry = y - s->cy;
    const double lx = rx * s->cos_a + ry * s->sin_a;
    const double ly = -rx * s->sin_a + ry * s->cos_a;
    double qx = fabs(lx) - s->hx, qy = fabs(ly) - s->hy, qz = fabs(z - s->cz) - s->hz;
    if (qx < 0.0) qx = 0.0;
    if (qy < 0.0) qy = 0.0;
    if (qz < 0.0) qz = 0.0;
    return sqrt(qx * qx + qy * qy + qz * qz);
}

static Aabb prism_aabb(const SynthPrism* s) {
    Aabb a;
    const double ex = fabs(s->ax) * s->half_len + fabs(s->ay) * s->half_base;
    const double ey = fabs(s->ay) * s->half_len + fabs(s->ax) * s->half_base;
    a.lo[0] = s->cx - ex; a.hi[0] = s->cx + ex;
    a.lo[1] = s->cy - ey; a.hi[1] = s->cy + ey;
    a.lo[2] = s->z0; a.hi[2] = s->z0 + s->height;
    return a;
}

static Aabb box_aabb(const SynthBox* s) {
    Aabb a;
    const double ex = fabs(s->cos_a) * s->hx + fabs(s->sin_a) * s->hy;
    const double ey = fabs(s->sin_a) * s->hx + fabs(s->cos_a) * s->hy;
    a.lo[0] = s->cx - ex; a.hi[0] = s->cx + ex;
    a.lo[1] = s->cy - ey; a.hi[1] = s->cy + ey;
    a.lo[2] = s->cz - s->hz; a.hi[2] = s->cz + s->hz;
    return a;
}

static double aabb_gap(const Aabb* a, const Aabb* b) {
    double s = 0.0;
    for (int k = 0; k < 3; ++k) {
        double g = 0.0;
        if (a->hi[k] < b->lo[k]) g = b->lo[k] - a->hi[k];
        else if (b->hi[k] < a->lo[k]) g = a->lo[k] - b->hi[k];
        s += g * g;
    }
    return sqrt(s);
}

#define BLK 8

/* Fills out[nz][ny][nx]. Returns 0, or -1 on bad arguments / allocation. */
SYNTH_API int synth_eval(float* out, int nx, int ny, int nz, const float* mins, float cell,
                         int has_ground, float ground_z, const SynthPrism* prisms, int n_prisms,
                         const SynthBox* boxes, int n_boxes, float trunc, int nthreads) {
    if (!out || !mins || nx <= 0 || ny <= 0 || nz <= 0 || !(cell > 0.0f) || n_prisms < 0 ||
        n_boxes < 0 || (n_prisms && !prisms) || (n_boxes && !boxes))
        return -1;
    const int ns = n_prisms + n_boxes;
    Aabb* boxes_aabb = (Aabb*)malloc(sizeof(Aabb) * (size_t)(ns > 0 ? ns : 1));
    if (!boxes_aabb) return -1;
    for (int i = 0; i < n_prisms; ++i) boxes_aabb[i] = prism_aabb(&prisms[i]);
    for (int i = 0; i < n_boxes; ++i) boxes_aabb[n_prisms + i] = box_aabb(&boxes[i]);
    const int bnx = (nx + BLK - 1) / BLK, bny = (ny + BLK - 1) / BLK, bnz = (nz + BLK - 1) / BLK;
    const long long nblk = (long long)bnx * bny * bnz;
    int failed = 0;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        int* cand = (int*)malloc(sizeof(int) * (size_t)(ns > 0 ? ns : 1));
        if (!cand) {
#ifdef _OPENMP
#pragma omp atomic write
#endif
            failed = 1;
        }
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (long long b = 0; b < nblk; ++b) {
            if (!cand) continue;
            const int bz = (int)(b / ((long long)bnx * bny));
            const int by = (int)((b / bnx) % bny);
            const int bx = (int)(b % bnx);
            const int x0 = bx * BLK, y0 = by * BLK, z0 = bz * BLK;
            const int x1 = x0 + BLK < nx ? x0 + BLK : nx;
            const int y1 = y0 + BLK < ny ? y0 + BLK : ny;
            const int z1 = z0 + BLK < nz ? z0 + BLK : nz;
            /* the block's sample points span [first centre, last centre] */
            Aabb blk;
            blk.lo[0] = mins[0] + (x0 + 0.5) * cell; blk.hi[0] = mins[0] + (x1 - 0.5) * cell;
            blk.lo[1] = mins[1] + (y0 + 0.5) * cell; blk.hi[1] = mins[1] + (y1 - 0.5) * cell;
            blk.lo[2] = mins[2] + (z0 + 0.5) * cell; blk.hi[2] = mins[2] + (z1 - 0.5) * cell;
            const double cx = 0.5 * (blk.lo[0] + blk.hi[0]);
            const double cy = 0.5 * (blk.lo[1] + blk.hi[1]);
            const double cz = 0.5 * (blk.lo[2] + blk.hi[2]);
            const double hx = 0.5 * (blk.hi[0] - blk.lo[0]);
            const double hy = 0.5 * (blk.hi[1] - blk.lo[1]);
            const double hz = 0.5 * (blk.hi[2] - blk.lo[2]);
            const double rad = sqrt(hx * hx + hy * hy + hz * hz);
            double best = (double)trunc;
            if (has_ground) {
                const double g = cz - ground_z > 0.0 ? cz - ground_z : 0.0;
                if (g < best) best = g;
            }
            for (int i = 0; i < n_prisms; ++i) {
                const double d = prism_dist(&prisms[i], cx, cy, cz);
                if (d < best) best = d;
            }
            for (int i = 0; i < n_boxes; ++i) {
                const double d = box_dist(&boxes[i], cx, cy, cz);
                if (d < best) best = d;
            }
            const double ub = best + rad;
            int nc = 0;
            for (int i = 0; i < ns; ++i)
                if (aabb_gap(&blk, &boxes_aabb[i]) <= ub) cand[nc++] = i;
            for (int iz = z0; iz < z1; ++iz) {
                const float pz = mins[2] + ((float)iz + 0.5f) * cell;
                for (int iy = y0; iy < y1; ++iy) {
                    const float py = mins[1] + ((float)iy + 0.5f) * cell;
                    for (int ix = x0; ix < x1; ++ix) {
                        const float px = mins[0] + ((float)ix + 0.5f) * cell;
                        double d = (double)trunc;
                        if (has_ground) {
                            const double g = (double)pz - ground_z > 0.0 ? (double)pz - ground_z : 0.0;
                            if (g < d) d = g;
                        }
                        for (int k = 0; k < nc && d > 0.0; ++k) {
                            const int i = cand[k];
                            const double e = i < n_prisms ? prism_dist(&prisms[i], px, py, pz)
                                                          : box_dist(&boxes[i - n_prisms], px, py, pz);
                            if (e < d) d = e;
                        }
                        out[((size_t)iz * ny + iy) * nx + ix] = (float)d;
                    }
                }
            }
        }
        free(cand);
    }
    free(boxes_aabb);
    return failed ? -1 : 0;
}

/* Reference implementation without culling, for tests of the culling. */
SYNTH_API int synth_eval_brute(float* out, int nx, int ny, int nz, const float* mins, float cell,
                               int has_ground, float ground_z, const SynthPrism* prisms,
                               int n_prisms, const SynthBox* boxes, int n_boxes, float trunc) {
    if (!out || !mins || nx <= 0 || ny <= 0 || nz <= 0) return -1;
    for (int iz = 0; iz < nz; ++iz)
        for (int iy = 0; iy < ny; ++iy)
            for (int ix = 0; ix < nx; ++ix) {
                const float px = mins[0] + ((float)ix + 0.5f) * cell;
                const float py = mins[1] + ((float)iy + 0.5f) * cell;
                const float pz = mins[2] + ((float)iz + 0.5f) * cell;
                double d = (double)trunc;
                if (has_ground) {
                    const double g = (double)pz - ground_z > 0.0 ? (double)pz - ground_z : 0.0;
                    if (g < d) d = g;
                }
                for (int i = 0; i < n_prisms; ++i) {
                    const double e = prism_dist(&prisms[i], px, py, pz);
                    if (e < d) d = e;
                }
                for (int i = 0; i < n_boxes; ++i) {
                    const double e = box_dist(&boxes[i], px, py, pz);
                    if (e < d) d = e;
                }
                out[((size_t)iz * ny + iy) * nx + ix] = (float)d;
            }
    return 0;
}

/* Point queries (for pose sampling and tests). xyz is [n][3]. */
SYNTH_API void synth_query(const float* xyz, int n, int has_ground, float ground_z,
                           const SynthPrism* prisms, int n_prisms, const SynthBox* boxes,
                           int n_boxes, float trunc, float* out) {
    for (int j = 0; j < n; ++j) {
        const double x = xyz[3 * j], y = xyz[3 * j + 1], z = xyz[3 * j + 2];
        double d = (double)trunc;
        if (has_ground) {
            const double g = z - ground_z > 0.0 ? z - ground_z : 0.0;
            if (g < d) d = g;
        }
        for (int i = 0; i < n_prisms; ++i) {
            const double e = prism_dist(&prisms[i], x, y, z);
            if (e < d) d = e;
        }
        for (int i = 0; i < n_boxes; ++i) {
            const double e = box_dist(&boxes[i], x, y, z);
            if (e < d) d = e;
        }
        out[j] = (float)d;
    }
}
