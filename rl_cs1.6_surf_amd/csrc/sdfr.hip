// sdfr.hip — MI355X (gfx950) SDF depth renderer: kernels and the C ABI of
// include/sdfr.h.
//
// The path it replaces is the reference's per-tick lidar render,
// python/surfgym/vision.py: GpuLidar._render_triton (:552-594) launching
// _march_kernel (:59-116), whose CPU twin is _render_torch (:626-666).
//
// Per ray (n, r, c) of env n, image row r, column c:
//   eye   = origin[n] + (0, 0, ducked[n] ? 12 : 17)              (vision.py:77-78)
//   yaw   = f32(yaw_deg[n] * f32(pi/180)) + yoff[c]               (vision.py:79, 586)
//   pitch = f32(pitch_deg[n] * f32(pi/180)) + poff[r]             (vision.py:80, 586)
//   dir   = (cos p cos y, cos p sin y, sin p)                     (vision.py:81-84)
//   march: t = 0; for k < max_steps while alive:                  (vision.py:100-111)
//            i_a = clamp(trunc(((eye_a + dir_a*t) - mins_a) * inv_cell), 0, n_a-1)
//            s = grid[iz][iy][ix]
//            alive = s > hit_eps && t < range
//            t += alive ? max(0.9*s, min_step) : 0
//   t = min(t, range); enc = min(t,near)/near + 0.25*(1-exp(-max(t-near,0)/2500))
//
// Arithmetic is fp32 in the order the reference's CPU path evaluates it,
// without FMA contraction (the file is compiled with -ffp-contract=off), so
// the march reproduces a faithful CPU evaluation step for step. cos/sin/exp
// are evaluated in fp64 and rounded once to fp32, which gives the correctly
// rounded fp32 value except in cases rarer than 1 in 2^28.
//
// Work decomposition. One wave64 owns a 2-D tile of pixels of one env (8x8
// by default): neighbouring pixels cast nearly parallel rays from the same
// eye, so the 64 lanes' gathers fall on few cache lines and the wave's loop
// trip count (its slowest ray) stays close to its mean ray. Blocks are
// re-numbered so that each XCD (blocks are dealt to the 8 XCDs round-robin)
// works on a contiguous run of envs, keeping an env's tiles in one L2.

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdarg.h>
#include <stdint.h>
#include <string.h>
#include <stdio.h>
#include <math.h>

#include "../../include/sdfr.h"

namespace {

constexpr double kD2R = 3.14159265358979323846 / 180.0;  // np.pi / 180.0 in float64
constexpr float kD2Rf = (float)kD2R;                      // the fp32 scalar torch multiplies by

// ---------------------------------------------------------------- errors --
thread_local char g_err[512];

__attribute__((format(printf, 2, 3))) int32_t fail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

// ---------------------------------------------------------------- handle --
}  // namespace

struct SdfrGrid {
    SdfrGridDesc desc;
    int32_t store_dtype;   // SDFR_F32 | SDFR_F16
    int32_t layout;        // SDFR_LAYOUT_*
    int32_t bx, by, bz;    // brick counts (BRICK4), else nx, ny, nz
    void* data;            // device copy
    int64_t bytes;
    int device;
};

namespace {

// ------------------------------------------------------------ grid access --
template <int LAYOUT>
__device__ __forceinline__ uint32_t voxel_index(int ix, int iy, int iz, int nx, int ny,
                                                int bx, int by) {
    if constexpr (LAYOUT == SDFR_LAYOUT_LINEAR) {
        return ((uint32_t)iz * (uint32_t)ny + (uint32_t)iy) * (uint32_t)nx + (uint32_t)ix;
    } else {
        uint32_t brick = (((uint32_t)(iz >> 2) * (uint32_t)by) + (uint32_t)(iy >> 2)) * (uint32_t)bx
                         + (uint32_t)(ix >> 2);
        uint32_t inner = ((uint32_t)(iz & 3) << 4) | ((uint32_t)(iy & 3) << 2) | (uint32_t)(ix & 3);
        return (brick << 6) | inner;
    }
}

__device__ __forceinline__ float load_voxel(const float* g, uint32_t i) { return g[i]; }
__device__ __forceinline__ float load_voxel(const __half* g, uint32_t i) { return __half2float(g[i]); }

// ------------------------------------------------------------- conversions --
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);   // encodings are finite and non-negative
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ bool read_ducked(const void* p, int64_t i, int dtype) {
    switch (dtype) {
        case SDFR_F32: return ((const float*)p)[i] != 0.0f;
        case SDFR_F64: return ((const double*)p)[i] != 0.0;
        case SDFR_I32: return ((const int32_t*)p)[i] != 0;
        case SDFR_I64: return ((const int64_t*)p)[i] != 0;
        case SDFR_U8: return ((const uint8_t*)p)[i] != 0;
        default: return (((const uint16_t*)p)[i] & 0x7fffu) != 0;  // f16 / bf16
    }
}

// Per-pixel camera offsets, float64 then rounded, term for term as the
// reference builds its tables (vision.py:502-509 equiangular, :515-526 pinhole).
__device__ __forceinline__ float equiangular_offset(int i, int n, double fov_deg) {
    double a = (double)i + 0.5;
    a = a / (double)n;
    a = 0.5 - a;
    a = fov_deg * a;
    a = a * kD2R;
    return (float)a;
}

__device__ __forceinline__ float pinhole_u(int c, int w, double tan_half) {
    if (w == 1) return 0.0f;
    double a = 2.0 * (double)c;
    a = a / (double)(w - 1);
    a = a - 1.0;
    return (float)(tan_half * a);
}

__device__ __forceinline__ float pinhole_v(int r, int h, double tan_half) {
    if (h == 1) return 0.0f;
    double a = 2.0 * (double)r;
    a = a / (double)(h - 1);
    a = 1.0 - a;
    return (float)(tan_half * a);
}

__device__ __forceinline__ void sincos_f32(float x, float* s, float* c) {
    double sd, cd;
    sincos((double)x, &sd, &cd);
    *s = (float)sd;
    *c = (float)cd;
}

// --------------------------------------------------------------- the args --
struct MarchArgs {
    const void* grid;
    int nx, ny, nz, bx, by;
    float fnx1, fny1, fnz1;       // n-1 as float: the clamp bound
    float mnx, mny, mnz, inv_cell;
    float rng, near, hit_eps, min_step;
    int max_steps;
    int W, H, camera;
    double hfov, vfov, tan_h, tan_v;
    const float* origin; int64_t origin_stride;
    const float* yaw; int64_t yaw_stride;
    const float* pitch; int64_t pitch_stride;
    const void* ducked; int64_t ducked_stride; int ducked_dtype;
    void* out; int64_t env_stride;
    int32_t* taps;
    int tiles_x, tiles_per_env;
    int64_t total_tiles;
    int nblocks;
};

// Block b runs on XCD b % 8; give XCD x the x-th contiguous eighth of the
// logical blocks (a bijection for any block count).
__device__ __forceinline__ int xcd_logical_block(int b, int nblocks) {
    int q = nblocks >> 3, rem = nblocks & 7;
    int x = b & 7, i = b >> 3;
    return x * q + (x < rem ? x : rem) + i;
}

// -------------------------------------------------------------- ray setup --
struct Ray {
    float ex, ey, ez, dx, dy, dz;
};

// Eye and unit direction of ray (n, r, c): vision.py:68-84 (kernel) and
// :596-624 (the CPU path's _dirs_equiangular / _dirs_pinhole).
__device__ __forceinline__ Ray make_ray(const MarchArgs& a, int n, int r, int c) {
    Ray ray;
    const float ox = a.origin[n * a.origin_stride + 0];
    const float oy = a.origin[n * a.origin_stride + 1];
    const float oz = a.origin[n * a.origin_stride + 2];
    const float yr = a.yaw[n * a.yaw_stride] * kD2Rf;
    const float pr = a.pitch[n * a.pitch_stride] * kD2Rf;
    const bool dk = read_ducked(a.ducked, n * a.ducked_stride, a.ducked_dtype);
    ray.ex = ox;
    ray.ey = oy;
    ray.ez = oz + (dk ? 12.0f : 17.0f);
    if (a.camera == SDFR_CAM_EQUIANGULAR) {
        const float yw = yr + equiangular_offset(c, a.W, a.hfov);
        const float pt = pr + equiangular_offset(r, a.H, a.vfov);
        float sp, cp, sy, cy;
        sincos_f32(pt, &sp, &cp);
        sincos_f32(yw, &sy, &cy);
        ray.dx = cp * cy;
        ray.dy = cp * sy;
        ray.dz = sp;
    } else {
        const float u = pinhole_u(c, a.W, a.tan_h);
        const float v = pinhole_v(r, a.H, a.tan_v);
        float sp, cp, sy, cy;
        sincos_f32(pr, &sp, &cp);
        sincos_f32(yr, &sy, &cy);
        // forward + u*right + v*up, then normalised (the CPU path's rsqrt is
        // 1/sqrt with two fp32 roundings)
        const float px = cp * cy + u * sy - v * sp * cy;
        const float py = cp * sy - u * cy - v * sp * sy;
        const float pz = sp + v * cp;
        const float inv = 1.0f / sqrtf(px * px + py * py + pz * pz);
        ray.dx = px * inv;
        ray.dy = py * inv;
        ray.dz = pz * inv;
    }
    return ray;
}

// The encoding, vision.py:112-116 / :654-657; t already clamped to range.
__device__ __forceinline__ float encode_depth(float t, float near) {
    const float lin = fminf(t, near) / near;
    const float xe = -fmaxf(t - near, 0.0f) / 2500.0f;
    const float ed = (float)exp((double)xe);
    return lin + 0.25f * (1.0f - ed);
}

// ------------------------------------------------------------- the kernel --
template <typename GT, int LAYOUT, int OUT_DTYPE, int TW, int TH, bool CENSUS>
__global__ __launch_bounds__(256) void march_tiles(MarchArgs a) {
    static_assert(TW * TH == 64, "one wave64 per tile");
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int blk = xcd_logical_block(blockIdx.x, a.nblocks);
    const int64_t tile = (int64_t)blk * 4 + wave;
    if (tile >= a.total_tiles) return;
    const int n = (int)(tile / a.tiles_per_env);
    const int rem = (int)(tile - (int64_t)n * a.tiles_per_env);
    const int ty = rem / a.tiles_x, tx = rem - ty * a.tiles_x;
    const int r = ty * TH + lane / TW;
    const int c = tx * TW + lane % TW;
    if (r >= a.H || c >= a.W) return;

    const Ray ray = make_ray(a, n, r, c);
    const GT* __restrict__ g = (const GT*)a.grid;
    float t = 0.0f;
    int taps = 0;
    for (int k = 0; k < a.max_steps; ++k) {
        const float px = ray.ex + ray.dx * t;
        const float py = ray.ey + ray.dy * t;
        const float pz = ray.ez + ray.dz * t;
        const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
        const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
        const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
        const float s = load_voxel(g, voxel_index<LAYOUT>(ix, iy, iz, a.nx, a.ny, a.bx, a.by));
        if constexpr (CENSUS) ++taps;
        if (!(s > a.hit_eps) || !(t < a.rng)) break;
        t = t + fmaxf(s * 0.9f, a.min_step);
    }
    const float enc = encode_depth(fminf(t, a.rng), a.near);

    const int64_t o = (int64_t)n * a.env_stride + (int64_t)r * a.W + c;
    if constexpr (OUT_DTYPE == SDFR_BF16) {
        ((uint16_t*)a.out)[o] = f32_to_bf16_rne(enc);
    } else {
        ((float*)a.out)[o] = enc;
    }
    if constexpr (CENSUS) a.taps[((int64_t)n * a.H + r) * a.W + c] = taps;
}

// One thread per ray: the directions make_ray() casts, (N,H,W,3) f32.
__global__ __launch_bounds__(256) void ray_dirs_kernel(MarchArgs a, float* dirs, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t hw = (int64_t)a.W * a.H;
    const int n = (int)(i / hw);
    const int pix = (int)(i - (int64_t)n * hw);
    const int r = pix / a.W, c = pix - r * a.W;
    const Ray ray = make_ray(a, n, r, c);
    dirs[3 * i + 0] = ray.dx;
    dirs[3 * i + 1] = ray.dy;
    dirs[3 * i + 2] = ray.dz;
}

// ------------------------------------------------------------- grid build --
template <typename ST, typename DT, int LAYOUT>
__global__ __launch_bounds__(256) void relayout_grid(const ST* __restrict__ src, DT* __restrict__ dst,
                                                      int nx, int ny, int nz, int bx, int by,
                                                      int64_t dst_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= dst_count) return;
    int ix, iy, iz;
    if constexpr (LAYOUT == SDFR_LAYOUT_LINEAR) {
        ix = (int)(i % nx);
        iy = (int)((i / nx) % ny);
        iz = (int)(i / ((int64_t)nx * ny));
    } else {
        const int64_t brick = i >> 6;
        const int inner = (int)(i & 63);
        const int64_t bxy = (int64_t)bx * by;
        const int bz_i = (int)(brick / bxy);
        const int by_i = (int)((brick % bxy) / bx);
        const int bx_i = (int)(brick % bx);
        ix = bx_i * 4 + (inner & 3);
        iy = by_i * 4 + ((inner >> 2) & 3);
        iz = bz_i * 4 + (inner >> 4);
    }
    float v = 0.0f;   // padding voxels are never addressed (indices clamp to n-1)
    if (ix < nx && iy < ny && iz < nz) {
        const int64_t s = ((int64_t)iz * ny + iy) * nx + ix;
        if constexpr (sizeof(ST) == 2) v = __half2float(((const __half*)src)[s]);
        else v = ((const float*)src)[s];
    }
    if constexpr (sizeof(DT) == 2) ((__half*)dst)[i] = __float2half_rn(v);
    else ((float*)dst)[i] = v;
}

template <typename ST, typename DT>
hipError_t launch_relayout(const void* src, void* dst, const SdfrGrid* g, int64_t count,
                           hipStream_t st) {
    const int blocks = (int)((count + 255) / 256);
    if (g->layout == SDFR_LAYOUT_LINEAR)
        relayout_grid<ST, DT, SDFR_LAYOUT_LINEAR><<<blocks, 256, 0, st>>>(
            (const ST*)src, (DT*)dst, g->desc.nx, g->desc.ny, g->desc.nz, g->bx, g->by, count);
    else
        relayout_grid<ST, DT, SDFR_LAYOUT_BRICK4><<<blocks, 256, 0, st>>>(
            (const ST*)src, (DT*)dst, g->desc.nx, g->desc.ny, g->desc.nz, g->bx, g->by, count);
    return hipGetLastError();
}

// --------------------------------------------------------- render dispatch --
template <typename GT, int LAYOUT, int OUT, bool CENSUS>
void launch_march(const MarchArgs& a, hipStream_t st) {
    march_tiles<GT, LAYOUT, OUT, 8, 8, CENSUS><<<a.nblocks, 256, 0, st>>>(a);
}

template <typename GT, int LAYOUT>
void dispatch_out(const MarchArgs& a, int out_dtype, bool census, hipStream_t st) {
    if (out_dtype == SDFR_BF16) {
        if (census) launch_march<GT, LAYOUT, SDFR_BF16, true>(a, st);
        else launch_march<GT, LAYOUT, SDFR_BF16, false>(a, st);
    } else {
        if (census) launch_march<GT, LAYOUT, SDFR_F32, true>(a, st);
        else launch_march<GT, LAYOUT, SDFR_F32, false>(a, st);
    }
}

bool dtype_ok_for_ducked(int d) {
    return d == SDFR_F32 || d == SDFR_F16 || d == SDFR_BF16 || d == SDFR_I32 || d == SDFR_I64 ||
           d == SDFR_U8 || d == SDFR_F64;
}

void copy_err(char* err, int32_t errlen) {
    if (err && errlen > 0) {
        strncpy(err, g_err, (size_t)errlen - 1);
        err[errlen - 1] = '\0';
    }
}

int32_t check_cam_poses(const char* fn, const SdfrCam* cam, const SdfrPoses* poses) {
    if (!cam || !poses) return fail(-1, "%s: null camera or poses argument", fn);
    if (cam->width <= 0 || cam->height <= 0)
        return fail(-2, "%s: image size must be positive (got %d x %d)", fn, cam->width,
                    cam->height);
    if ((int64_t)cam->width * cam->height > (1 << 24))
        return fail(-2, "%s: image too large (%lld pixels, limit 2^24)", fn,
                    (long long)cam->width * cam->height);
    if (cam->max_steps < 0) return fail(-2, "%s: max_steps must be >= 0 (got %d)", fn, cam->max_steps);
    if (!(cam->near > 0.0f)) return fail(-2, "%s: near must be > 0", fn);
    if (cam->camera != SDFR_CAM_EQUIANGULAR && cam->camera != SDFR_CAM_PINHOLE)
        return fail(-3, "%s: unknown camera model %d", fn, cam->camera);
    if (poses->n_envs <= 0) return fail(-2, "%s: n_envs must be >= 1 (got %d)", fn, poses->n_envs);
    if (!poses->origin || !poses->yaw_deg || !poses->pitch_deg || !poses->ducked)
        return fail(-1, "%s: null pose pointer", fn);
    if (!dtype_ok_for_ducked(poses->ducked_dtype))
        return fail(-3, "%s: unsupported ducked dtype %d", fn, poses->ducked_dtype);
    return 0;
}

void fill_args(MarchArgs* a, const SdfrCam* cam, const SdfrPoses* poses) {
    memset(a, 0, sizeof *a);
    a->rng = cam->range;
    a->near = cam->near;
    a->hit_eps = cam->hit_eps;
    a->min_step = cam->min_step;
    a->max_steps = cam->max_steps;
    a->W = cam->width;
    a->H = cam->height;
    a->camera = cam->camera;
    a->hfov = cam->hfov_deg;
    a->vfov = cam->vfov_deg;
    a->tan_h = cam->tan_half_h;
    a->tan_v = cam->tan_half_v;
    a->origin = poses->origin;
    a->origin_stride = poses->origin_stride;
    a->yaw = poses->yaw_deg;
    a->yaw_stride = poses->yaw_stride;
    a->pitch = poses->pitch_deg;
    a->pitch_stride = poses->pitch_stride;
    a->ducked = poses->ducked;
    a->ducked_stride = poses->ducked_stride;
    a->ducked_dtype = poses->ducked_dtype;
}

}  // namespace

// ================================================================ C ABI ==
extern "C" {

SDFR_API int32_t sdfr_abi_version(void) { return SDFR_ABI_VERSION; }

SDFR_API const char* sdfr_last_error(void) { return g_err; }

SDFR_API int64_t sdfr_grid_bytes(const SdfrGrid* grid) { return grid ? grid->bytes : -1; }

SDFR_API SdfrGrid* sdfr_grid_create(const SdfrGridDesc* desc, const void* src, int32_t src_dtype,
                                    int32_t src_on_device, int32_t store_dtype, int32_t layout,
                                    void* stream, char* err, int32_t errlen) {
    g_err[0] = '\0';
    if (!desc || !src) {
        fail(-1, "sdfr_grid_create: null descriptor or source");
        copy_err(err, errlen);
        return nullptr;
    }
    if (desc->nx <= 0 || desc->ny <= 0 || desc->nz <= 0) {
        fail(-2, "sdfr_grid_create: grid dims must be positive (got %d x %d x %d)",
             desc->nx, desc->ny, desc->nz);
        copy_err(err, errlen);
        return nullptr;
    }
    if (!(desc->cell > 0.0f) || !isfinite(desc->cell)) {
        fail(-2, "sdfr_grid_create: cell must be a positive finite size");
        copy_err(err, errlen);
        return nullptr;
    }
    if (src_dtype != SDFR_F32 && src_dtype != SDFR_F16) {
        fail(-3, "sdfr_grid_create: source dtype must be f32 or f16 (got %d)", src_dtype);
        copy_err(err, errlen);
        return nullptr;
    }
    if (store_dtype != SDFR_F32 && store_dtype != SDFR_F16) {
        fail(-3, "sdfr_grid_create: store dtype must be f32 or f16 (got %d)", store_dtype);
        copy_err(err, errlen);
        return nullptr;
    }
    if (layout != SDFR_LAYOUT_LINEAR && layout != SDFR_LAYOUT_BRICK4) {
        fail(-3, "sdfr_grid_create: unknown layout %d", layout);
        copy_err(err, errlen);
        return nullptr;
    }
    const int64_t nvox = (int64_t)desc->nx * desc->ny * desc->nz;
    int bx = desc->nx, by = desc->ny, bz = desc->nz;
    int64_t count = nvox;
    if (layout == SDFR_LAYOUT_BRICK4) {
        bx = (desc->nx + 3) / 4;
        by = (desc->ny + 3) / 4;
        bz = (desc->nz + 3) / 4;
        count = (int64_t)bx * by * bz * 64;
    }
    if (count >= ((int64_t)1 << 32)) {
        fail(-2, "sdfr_grid_create: grid too large (%lld voxels, limit 2^32)", (long long)count);
        copy_err(err, errlen);
        return nullptr;
    }

    hipStream_t st = (hipStream_t)stream;
    SdfrGrid* g = new SdfrGrid();
    g->desc = *desc;
    g->store_dtype = store_dtype;
    g->layout = layout;
    g->bx = bx;
    g->by = by;
    g->bz = bz;
    g->bytes = count * (store_dtype == SDFR_F16 ? 2 : 4);
    g->data = nullptr;
    (void)hipGetDevice(&g->device);

    const int64_t src_bytes = nvox * (src_dtype == SDFR_F16 ? 2 : 4);
    void* staged = nullptr;
    const void* dsrc = src;
    hipError_t e = hipMalloc(&g->data, (size_t)g->bytes);
    if (e == hipSuccess && !src_on_device) {
        e = hipMalloc(&staged, (size_t)src_bytes);
        if (e == hipSuccess)
            e = hipMemcpyAsync(staged, src, (size_t)src_bytes, hipMemcpyHostToDevice, st);
        dsrc = staged;
    }
    if (e == hipSuccess) {
        if (src_dtype == SDFR_F32 && store_dtype == SDFR_F32)
            e = launch_relayout<float, float>(dsrc, g->data, g, count, st);
        else if (src_dtype == SDFR_F32)
            e = launch_relayout<float, __half>(dsrc, g->data, g, count, st);
        else if (store_dtype == SDFR_F32)
            e = launch_relayout<__half, float>(dsrc, g->data, g, count, st);
        else
            e = launch_relayout<__half, __half>(dsrc, g->data, g, count, st);
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (staged) (void)hipFree(staged);
    if (e != hipSuccess) {
        fail(-4, "sdfr_grid_create: HIP error %s", hipGetErrorString(e));
        copy_err(err, errlen);
        if (g->data) (void)hipFree(g->data);
        delete g;
        return nullptr;
    }
    return g;
}

SDFR_API void sdfr_grid_destroy(SdfrGrid* grid) {
    if (!grid) return;
    if (grid->data) (void)hipFree(grid->data);
    delete grid;
}

SDFR_API int32_t sdfr_render(const SdfrGrid* grid, const SdfrCam* cam, const SdfrPoses* poses,
                             const SdfrImage* image, void* stream) {
    g_err[0] = '\0';
    if (!grid || !grid->data) return fail(-1, "sdfr_render: null grid handle");
    if (!image) return fail(-1, "sdfr_render: null image argument");
    int32_t rc = check_cam_poses("sdfr_render", cam, poses);
    if (rc) return rc;
    if (!image->out) return fail(-1, "sdfr_render: null output pointer");
    if (image->dtype != SDFR_F32 && image->dtype != SDFR_BF16)
        return fail(-3, "sdfr_render: output dtype must be f32 or bf16 (got %d)", image->dtype);
    if (image->env_stride < (int64_t)cam->width * cam->height)
        return fail(-2, "sdfr_render: env_stride %lld is smaller than H*W",
                    (long long)image->env_stride);

    MarchArgs a;
    fill_args(&a, cam, poses);
    a.grid = grid->data;
    a.nx = grid->desc.nx;
    a.ny = grid->desc.ny;
    a.nz = grid->desc.nz;
    a.bx = grid->bx;
    a.by = grid->by;
    a.fnx1 = (float)(grid->desc.nx - 1);
    a.fny1 = (float)(grid->desc.ny - 1);
    a.fnz1 = (float)(grid->desc.nz - 1);
    a.mnx = grid->desc.mins[0];
    a.mny = grid->desc.mins[1];
    a.mnz = grid->desc.mins[2];
    a.inv_cell = (float)(1.0 / (double)grid->desc.cell);   // Python's 1.0/cell, then fp32
    a.out = image->out;
    a.env_stride = image->env_stride;
    a.taps = image->taps;
    a.tiles_x = (cam->width + 7) / 8;
    a.tiles_per_env = a.tiles_x * ((cam->height + 7) / 8);
    a.total_tiles = (int64_t)a.tiles_per_env * poses->n_envs;
    const int64_t nblocks = (a.total_tiles + 3) / 4;
    if (nblocks > 0x7fffffff)
        return fail(-2, "sdfr_render: too many envs (%lld blocks)", (long long)nblocks);
    a.nblocks = (int)nblocks;

    hipStream_t st = (hipStream_t)stream;
    const bool census = image->taps != nullptr;
    if (grid->store_dtype == SDFR_F16) {
        if (grid->layout == SDFR_LAYOUT_BRICK4)
            dispatch_out<__half, SDFR_LAYOUT_BRICK4>(a, image->dtype, census, st);
        else
            dispatch_out<__half, SDFR_LAYOUT_LINEAR>(a, image->dtype, census, st);
    } else {
        if (grid->layout == SDFR_LAYOUT_BRICK4)
            dispatch_out<float, SDFR_LAYOUT_BRICK4>(a, image->dtype, census, st);
        else
            dispatch_out<float, SDFR_LAYOUT_LINEAR>(a, image->dtype, census, st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-4, "sdfr_render: launch failed: %s", hipGetErrorString(e));
    return 0;
}

SDFR_API int32_t sdfr_ray_dirs(const SdfrCam* cam, const SdfrPoses* poses, float* dirs,
                               void* stream) {
    g_err[0] = '\0';
    int32_t rc = check_cam_poses("sdfr_ray_dirs", cam, poses);
    if (rc) return rc;
    if (!dirs) return fail(-1, "sdfr_ray_dirs: null output pointer");
    MarchArgs a;
    fill_args(&a, cam, poses);
    const int64_t total = (int64_t)cam->width * cam->height * poses->n_envs;
    const int64_t blocks = (total + 255) / 256;
    if (blocks > 0x7fffffff) return fail(-2, "sdfr_ray_dirs: too many rays (%lld)", (long long)total);
    ray_dirs_kernel<<<(int)blocks, 256, 0, (hipStream_t)stream>>>(a, dirs, total);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-4, "sdfr_ray_dirs: launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
