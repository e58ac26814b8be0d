/* goal.c — CPU restatement of the reference's goal field. TEST
 * INFRASTRUCTURE ONLY: the oracle the GPU goal-field bake and sampler are
 * measured against, never part of the product path.
 *
 * oracle_goal_distance and oracle_goal_quantise follow
 * python/surfgym/goalfield.py:228-297: distance 0 on
 * the free voxels of the seed box, 26-neighbour relaxation
 *   d[v] = min(d[v], d[u] + w),  w = f32(cell * sqrt(|u - v|^2)),
 * in fp32 with solid voxels excluded, run to the fixpoint; reach_max = the
 * largest finite value; +inf -> sentinel = reach_max + 2*cell (fp64, stored
 * fp32); q = clamp(round_half_even(d * f32(1 / f32(cell/8))), 0, 65535).
 *
 * It reaches the fixpoint by Dijkstra's label-setting order rather than the
 * reference's Jacobi sweeps. Both give the same fp32 values: x -> fl(x + w) is
 * monotone and never below x, so the fixpoint is, for every voxel, the least
 * fp32 left-to-right path sum from a seed, and Dijkstra settles each voxel at
 * exactly that value. (tests/test_oracle_goal.py checks the two orders against
 * each other on random grids.)
 *
 * oracle_goal_sample follows GoalField.sample (goalfield.py:68-94) in its
 * numpy types: positions and grid coordinates in fp64, fractions, weights
 * and sums in fp32, honest corners v < f32(reach_max + cell/2).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define API __attribute__((visibility("default")))

typedef struct {
    float key;
    int64_t idx;
} Item;

typedef struct {
    Item* a;
    int64_t n, cap;
} Heap;

static int heap_push(Heap* h, float key, int64_t idx) {
    if (h->n == h->cap) {
        int64_t cap = h->cap ? 2 * h->cap : 1024;
        Item* a = (Item*)realloc(h->a, (size_t)cap * sizeof(Item));
        if (!a) return -1;
        h->a = a;
        h->cap = cap;
    }
    int64_t i = h->n++;
    while (i > 0) {
        int64_t p = (i - 1) / 2;
        if (h->a[p].key <= key) break;
        h->a[i] = h->a[p];
        i = p;
    }
    h->a[i].key = key;
    h->a[i].idx = idx;
    return 0;
}

static Item heap_pop(Heap* h) {
    Item top = h->a[0];
    Item last = h->a[--h->n];
    int64_t i = 0;
    for (;;) {
        int64_t c = 2 * i + 1;
        if (c >= h->n) break;
        if (c + 1 < h->n && h->a[c + 1].key < h->a[c].key) ++c;
        if (last.key <= h->a[c].key) break;
        h->a[i] = h->a[c];
        i = c;
    }
    if (h->n > 0) h->a[i] = last;
    return top;
}

/* Relaxed distances, +inf where unreachable or solid. Returns the number of
 * seed voxels (>= 0) or -1 on allocation failure. lo/hi: inclusive voxel box
 * (x, y, z), clipped here to the grid. */
API int64_t oracle_goal_distance(const uint8_t* occ, int nx, int ny, int nz, float cell,
                                 const int* lo_in, const int* hi_in, float* d) {
    const int64_t vox = (int64_t)nx * ny * nz;
    const int dims[3] = {nx, ny, nz};
    int lo[3], hi[3];
    for (int j = 0; j < 3; ++j) {
        lo[j] = lo_in[j] < 0 ? 0 : lo_in[j];
        hi[j] = hi_in[j] > dims[j] - 1 ? dims[j] - 1 : hi_in[j];
    }
    const float w[4] = {0.0f, (float)((double)cell * sqrt(1.0)), (float)((double)cell * sqrt(2.0)),
                        (float)((double)cell * sqrt(3.0))};
    for (int64_t i = 0; i < vox; ++i) d[i] = INFINITY;
    Heap h = {NULL, 0, 0};
    int64_t seeds = 0;
    for (int z = lo[2]; z <= hi[2]; ++z)
        for (int y = lo[1]; y <= hi[1]; ++y)
            for (int x = lo[0]; x <= hi[0]; ++x) {
                const int64_t i = ((int64_t)z * ny + y) * nx + x;
                if (occ[i]) continue;
                d[i] = 0.0f;
                ++seeds;
                if (heap_push(&h, 0.0f, i)) {
                    free(h.a);
                    return -1;
                }
            }
    while (h.n > 0) {
        const Item it = heap_pop(&h);
        if (it.key > d[it.idx]) continue;   /* stale entry */
        const int64_t i = it.idx;
        const int x = (int)(i % nx), y = (int)((i / nx) % ny), z = (int)(i / ((int64_t)nx * ny));
        for (int oz = -1; oz <= 1; ++oz)
            for (int oy = -1; oy <= 1; ++oy)
                for (int ox = -1; ox <= 1; ++ox) {
                    const int q = oz * oz + oy * oy + ox * ox;
                    if (q == 0) continue;
                    const int ux = x + ox, uy = y + oy, uz = z + oz;
                    if (ux < 0 || uy < 0 || uz < 0 || ux >= nx || uy >= ny || uz >= nz) continue;
                    const int64_t u = ((int64_t)uz * ny + uy) * nx + ux;
                    if (occ[u]) continue;
                    const float nd = it.key + w[q];
                    if (nd < d[u]) {
                        d[u] = nd;
                        if (heap_push(&h, nd, u)) {
                            free(h.a);
                            return -1;
                        }
                    }
                }
    }
    free(h.a);
    return seeds;
}

/* From relaxed distances to the stored field. Returns 0, or -6 when the
 * sentinel does not fit the uint16 range (goalfield.py:279-290). */
API int oracle_goal_quantise(const float* d, int64_t vox, float cell, uint16_t* q_out, float* g_out,
                             float* reach_out, float* sentinel_out, float* quant_out) {
    float reach = 0.0f;
    for (int64_t i = 0; i < vox; ++i)
        if (d[i] != INFINITY && d[i] > reach) reach = d[i];
    const double sentinel = (double)reach + 2.0 * (double)cell;
    const double quant = (double)cell / 8.0;
    *reach_out = reach;
    *sentinel_out = (float)sentinel;
    *quant_out = (float)quant;
    if (sentinel / quant > 65535.0) return -6;
    const float sent_f = (float)sentinel, quant_f = (float)quant;
    const float inv = 1.0f / quant_f;
    for (int64_t i = 0; i < vox; ++i) {
        float v = d[i] == INFINITY ? sent_f : d[i];
        float q = nearbyintf(v * inv);
        q = q < 0.0f ? 0.0f : (q > 65535.0f ? 65535.0f : q);
        const uint16_t u = (uint16_t)q;
        if (q_out) q_out[i] = u;
        if (g_out) g_out[i] = (float)u * quant_f;
    }
    return 0;
}

API void oracle_goal_sample(const float* grid, int nx, int ny, int nz, const double* mins,
                            double cell, double reach_max, const double* pos, int64_t n, float* out) {
    const float valid_max = (float)(reach_max + 0.5 * cell);
    const float sentinel = (float)(reach_max + 2.0 * cell);
    const int dims[3] = {nx, ny, nz};
    for (int64_t i = 0; i < n; ++i) {
        int64_t i0[3];
        float f[3];
        for (int j = 0; j < 3; ++j) {
            const double g = (pos[3 * i + j] - mins[j]) / cell - 0.5;
            const double fl = floor(g);
            i0[j] = (int64_t)fl;
            f[j] = (float)(g - (double)i0[j]);
        }
        float num = 0.0f, den = 0.0f;
        for (int dz = 0; dz < 2; ++dz)
            for (int dy = 0; dy < 2; ++dy)
                for (int dx = 0; dx < 2; ++dx) {
                    const int dd[3] = {dx, dy, dz};
                    int64_t c[3];
                    for (int j = 0; j < 3; ++j) {
                        int64_t v = i0[j] + dd[j];
                        c[j] = v < 0 ? 0 : (v > dims[j] - 1 ? dims[j] - 1 : v);
                    }
                    const float v = grid[(c[2] * ny + c[1]) * nx + c[0]];
                    const float wx = dx ? f[0] : 1.0f - f[0];
                    const float wy = dy ? f[1] : 1.0f - f[1];
                    const float wz = dz ? f[2] : 1.0f - f[2];
                    const float wgt = wx * wy * wz * (v < valid_max ? 1.0f : 0.0f);
                    num += wgt * v;
                    den += wgt;
                }
        out[i] = den > 1e-6f ? num / (den > 1e-6f ? den : 1e-6f) : sentinel;
    }
}
