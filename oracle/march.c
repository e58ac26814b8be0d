/* oracle/march.c — CPU restatement of the reference's SDF depth render.
 *
 * TEST INFRASTRUCTURE ONLY. This is the oracle the GPU renderer is compared
 * against; only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline
 * leg may load it. The product path never calls it.
 *
 * It restates, per ray, what python/surfgym/vision.py computes in
 * _render_torch (:626-666) with the direction setup of _dirs_equiangular
 * (:596-607) / _dirs_pinhole (:609-624), the tables of GpuLidar.__init__
 * (:499-529), and the march semantics of _march_kernel (:85-116):
 *
 *   eye.z = origin.z + (ducked ? 12 : 17)                  vision.py:633, :77-78
 *   yr = f32(yaw_deg * f32(pi/180)), pr likewise            vision.py:603-604, :586
 *   equiangular: y = yr + yoff[c], p = pr + poff[r]          vision.py:603-607
 *                d = (cos p cos y, cos p sin y, sin p)
 *   pinhole:     d = normalise(fwd + u*right + v*up)          vision.py:614-624
 *   loop k < max_steps:                                       vision.py:642-653
 *       i_a = clamp(trunc(((e_a + d_a*t) - mins_a) * inv_cell), 0, n_a-1)
 *       s = grid[(iz*ny + iy)*nx + ix]
 *       alive = alive && s > hit_eps && t < range
 *       t += alive ? max(s*0.9, min_step) : 0
 *   t = min(t, range)                                         vision.py:654
 *   enc = min(t,near)/near + 0.25*(1 - exp(-max(t-near,0)/2500))  vision.py:655-657
 *
 * Lockstep over all rays (the reference's CPU loop) and a per-ray loop that
 * stops when the ray dies give identical results: `alive` only ever turns
 * off and a dead ray adds exactly 0 to t (vision.py:91-98). This file uses
 * the per-ray form and also reports the number of grid loads each ray
 * issued (the census of tools/bench_lidar.py:45-88, counting loads).
 *
 * Arithmetic: fp32, evaluated in the reference's operation order, one
 * rounding per operation (build with -ffp-contract=off, no fast-math; x86-64
 * SSE arithmetic is IEEE single). cos/sin/exp are taken in double and rounded
 * once to float, i.e. the correctly rounded fp32 value in all but rare ties.
 * The camera tables are float64 then rounded, as numpy builds them.
 */
#include <math.h>
#include <stdint.h>
#include <stddef.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_API __attribute__((visibility("default")))

static const double D2R = 3.14159265358979323846 / 180.0;   /* np.pi / 180.0 */

/* GpuLidar.__init__ equiangular tables, vision.py:502-509 */
ORACLE_API float oracle_equiangular_offset(int i, int n, double fov_deg) {
    double a = (double)i + 0.5;
    a = a / (double)n;
    a = 0.5 - a;
    a = fov_deg * a;
    a = a * D2R;
    return (float)a;
}

/* GpuLidar.__init__ pinhole tables, vision.py:515-526 */
ORACLE_API float oracle_pinhole_u(int c, int w, double tan_half) {
    if (w == 1) return 0.0f;
    double a = 2.0 * (double)c;
    a = a / (double)(w - 1);
    a = a - 1.0;
    return (float)(tan_half * a);
}

ORACLE_API float oracle_pinhole_v(int r, int h, double tan_half) {
    if (h == 1) return 0.0f;
    double a = 2.0 * (double)r;
    a = a / (double)(h - 1);
    a = 1.0 - a;
    return (float)(tan_half * a);
}

static inline float f_cos(float x) { return (float)cos((double)x); }
static inline float f_sin(float x) { return (float)sin((double)x); }

/* Unit direction of ray (r, c) for one env, both camera models. */
ORACLE_API void oracle_ray_dir(int camera, int r, int c, int W, int H, double hfov, double vfov,
                               double tan_h, double tan_v, float yaw_deg, float pitch_deg,
                               float* out3) {
    const float d2r = (float)D2R;
    const float yr = yaw_deg * d2r;
    const float pr = pitch_deg * d2r;
    if (camera == 0) {
        const float y = yr + oracle_equiangular_offset(c, W, hfov);
        const float p = pr + oracle_equiangular_offset(r, H, vfov);
        const float cp = f_cos(p);
        out3[0] = cp * f_cos(y);
        out3[1] = cp * f_sin(y);
        out3[2] = f_sin(p);
    } else {
        const float u = oracle_pinhole_u(c, W, tan_h);
        const float v = oracle_pinhole_v(r, H, tan_v);
        const float cy = f_cos(yr), sy = f_sin(yr), cp = f_cos(pr), sp = f_sin(pr);
        const float dx = cp * cy + u * sy - v * sp * cy;
        const float dy = cp * sy - u * cy - v * sp * sy;
        const float dz = sp + v * cp;
        const float inv = 1.0f / sqrtf(dx * dx + dy * dy + dz * dz);   /* torch.rsqrt on CPU */
        out3[0] = dx * inv;
        out3[1] = dy * inv;
        out3[2] = dz * inv;
    }
}

static inline int clamp_index(float f, int n) {
    /* .long() truncates toward zero, then clamp_(0, n-1) (vision.py:644-646) */
    if (!(f > 0.0f)) return 0;               /* negatives (and NaN) truncate/clamp to 0 */
    if (f >= (float)(n - 1)) return n - 1;
    return (int)f;
}

/* The encoding, vision.py:654-657 (t already clamped to range). */
ORACLE_API float oracle_encode(float t, float near) {
    const float lin = (t < near ? t : near) / near;
    float m = t - near;
    if (!(m > 0.0f)) m = 0.0f;
    const float x = -m / 2500.0f;
    const float e = (float)exp((double)x);
    return lin + 0.25f * (1.0f - e);
}

/* March one ray; returns the final (unclamped) t and the loads issued. */
ORACLE_API float oracle_march_ray(const float* grid, int nx, int ny, int nz, const float* mins,
                                  float inv_cell, float ex, float ey, float ez, float dx, float dy,
                                  float dz, float range, float hit_eps, float min_step,
                                  int max_steps, int32_t* loads) {
    float t = 0.0f;
    int k = 0, n_loads = 0;
    for (; k < max_steps; ++k) {
        const float px = ex + dx * t;
        const float py = ey + dy * t;
        const float pz = ez + dz * t;
        const int ix = clamp_index((px - mins[0]) * inv_cell, nx);
        const int iy = clamp_index((py - mins[1]) * inv_cell, ny);
        const int iz = clamp_index((pz - mins[2]) * inv_cell, nz);
        const float s = grid[((size_t)iz * (size_t)ny + (size_t)iy) * (size_t)nx + (size_t)ix];
        ++n_loads;
        if (!(s > hit_eps) || !(t < range)) break;
        const float st = s * 0.9f;
        t = t + (st > min_step ? st : min_step);
    }
    if (loads) *loads = n_loads;
    return t;
}

/* oracle_march_ray with a record of every sample it takes: for step k,
 * t_k[k] (the distance the sample is taken at), vox[3k..3k+2] (ix, iy, iz),
 * pos[3k..3k+2] (the unclamped voxel coordinates ((e + d*t) - mins) * inv_cell,
 * whose distance to the nearest integer is the sample's distance to a voxel
 * face in cells) and s_k[k] (the value read). Stores at most cap records;
 * returns the number of samples taken and writes the final t and the stop
 * reason (0 hit: s <= hit_eps, 1 range: t >= range, 2 steps exhausted). */
ORACLE_API int oracle_march_trace(const float* grid, int nx, int ny, int nz, const float* mins,
                                  float inv_cell, float ex, float ey, float ez, float dx, float dy,
                                  float dz, float range, float hit_eps, float min_step,
                                  int max_steps, int cap, float* t_k, int32_t* vox, float* pos,
                                  float* s_k, float* t_final, int32_t* why) {
    float t = 0.0f;
    int k = 0, reason = 2;
    for (; k < max_steps; ++k) {
        const float fx = ((ex + dx * t) - mins[0]) * inv_cell;
        const float fy = ((ey + dy * t) - mins[1]) * inv_cell;
        const float fz = ((ez + dz * t) - mins[2]) * inv_cell;
        const int ix = clamp_index(fx, nx), iy = clamp_index(fy, ny), iz = clamp_index(fz, nz);
        const float s = grid[((size_t)iz * (size_t)ny + (size_t)iy) * (size_t)nx + (size_t)ix];
        if (k < cap) {
            t_k[k] = t;
            vox[3 * k] = ix; vox[3 * k + 1] = iy; vox[3 * k + 2] = iz;
            pos[3 * k] = fx; pos[3 * k + 1] = fy; pos[3 * k + 2] = fz;
            s_k[k] = s;
        }
        if (!(s > hit_eps)) { reason = 0; ++k; break; }
        if (!(t < range)) { reason = 1; ++k; break; }
        const float st = s * 0.9f;
        t = t + (st > min_step ? st : min_step);
    }
    *t_final = t;
    *why = reason;
    return k;
}

/* Full render of N envs into out[N][H][W] (and loads[N][H][W] if given).
 * grid holds the voxel values exactly as the renderer reads them (an f16
 * store is emulated by the caller rounding to f16 and back). Poses are
 * dense: origin[N][3], yaw/pitch/ducked[N]. With nzg (the int8 |n_z|*127
 * surf-mask grid, same [nz][ny][nx] shape) the output is out[N][H][W][2]:
 * the depth encoding and |n_z| of the voxel the march stopped in, read at
 * the clamped t (vision.py:654-666). Returns 0, or -1 on bad args. */
ORACLE_API int oracle_render(const float* grid, int nx, int ny, int nz, const float* mins,
                             float cell, int W, int H, int camera, double hfov, double vfov,
                             double tan_h, double tan_v, float range, float near, float hit_eps,
                             float min_step, int max_steps, const float* origin, const float* yaw,
                             const float* pitch, const float* ducked, int N, float* out,
                             int32_t* loads, const int8_t* nzg, int nthreads) {
    if (!grid || !mins || !origin || !yaw || !pitch || !ducked || !out) return -1;
    if (nx <= 0 || ny <= 0 || nz <= 0 || W <= 0 || H <= 0 || N < 0 || !(near > 0.0f)) return -1;
    const float inv_cell = (float)(1.0 / (double)cell);
    const int ch = nzg ? 2 : 1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(dynamic, 1)
#endif
    for (long long job = 0; job < (long long)N * H; ++job) {
        const int n = (int)(job / H), r = (int)(job % H);
        const float ex = origin[3 * n + 0];
        const float ey = origin[3 * n + 1];
        const float ez = origin[3 * n + 2] + (ducked[n] != 0.0f ? 12.0f : 17.0f);
        for (int c = 0; c < W; ++c) {
            float d[3];
            oracle_ray_dir(camera, r, c, W, H, hfov, vfov, tan_h, tan_v, yaw[n], pitch[n], d);
            int32_t nl = 0;
            float t = oracle_march_ray(grid, nx, ny, nz, mins, inv_cell, ex, ey, ez, d[0], d[1],
                                       d[2], range, hit_eps, min_step, max_steps, &nl);
            t = t < range ? t : range;
            const size_t px = ((size_t)n * H + r) * W + c;
            out[px * ch] = oracle_encode(t, near);
            if (nzg) {
                const int ix = clamp_index(((ex + d[0] * t) - mins[0]) * inv_cell, nx);
                const int iy = clamp_index(((ey + d[1] * t) - mins[1]) * inv_cell, ny);
                const int iz = clamp_index(((ez + d[2] * t) - mins[2]) * inv_cell, nz);
                const int8_t v = nzg[((size_t)iz * (size_t)ny + (size_t)iy) * (size_t)nx + (size_t)ix];
                out[px * ch + 1] = (float)v / 127.0f;
            }
            if (loads) loads[px] = nl;
        }
    }
    return 0;
}
