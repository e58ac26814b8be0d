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
// One render is two or three launches on the caller's stream:
//   1. ray_setup: per env, the (sin, cos) of its H row pitch angles and W
//      column yaw angles, and its eye point — all the transcendental work of
//      ray setup, (H+W) fp64 sincos per env instead of two per ray;
//      With the lookahead tile order the same launch also keys the tiles by
//      where they look and counts them into buckets, and order_scatter
//      writes the sorted list (see "tile order");
//   2. the march, in one of three schedules with identical results:
//      - tiles (default): launch-scheduled two-wave workgroups, each wave
//        marching RPL 8x8 pixel tiles at once, RPL rays per lane (1 or 2,
//        chosen per render by render_rpl unless the caller fixes it);
//      - persistent: a grid that fills the GPU once; each wave keeps 64 ray
//        slots and refills finished slots with new rays (ray compaction),
//        pulling 8x8 pixel tiles from per-XCD work counters. It keeps every
//        lane busy but mixes rays of different depths in one gather, which
//        costs more cache lines per gather than it saves in idle lanes on
//        the scenes measured so far, so it is not the default;
//      - slots: persistent waves of R tile slots (see march_slots).
// Blocks are dealt to the 8 XCDs round-robin by the hardware; they are
// numbered so that each XCD works on a contiguous run of envs (env order), or
// on interleaved chunks of the sorted tile list (lookahead order), keeping
// rays that share grid data in one L2.

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/sdfr.h"

namespace {

constexpr double kD2R = 3.14159265358979323846 / 180.0;  // np.pi / 180.0 in float64
constexpr float kD2Rf = (float)kD2R;                      // the fp32 scalar torch multiplies by

// Raw buffer descriptor word 3 for gfx9-family (gfx950) untyped loads.
constexpr int32_t kRsrcWord3 = 0x00020000;
// Largest nx+ny+nz the per-workgroup axis tables hold (64 KiB of LDS).
constexpr int kMaxAxisEntries = 16384;
// Persistent schedule: 8 tile partitions (one per XCD) plus an exit counter,
// each in its own 128-byte line.
constexpr int kParts = 8;
constexpr int kCtrStride = 32;
constexpr int kCounterWords = (kParts + 1) * kCtrStride;
// Grids up to this size stay resident in the 256 MB Infinity Cache.
constexpr int64_t kCacheResidentBytes = 192ll << 20;
// On larger grids the march is bound by L2-miss traffic, and fewer rays in
// flight per XCD raise the L2 hit rate more than they cost in latency: the
// tiles schedule then holds at most this many workgroups per CU (by sizing
// their LDS), 24 waves instead of 32. Measured on a 1 GiB grid: 12 per CU
// 2.09 ms, 10 2.10, 16 (unlimited) 2.15, 5 2.55; on a cache-resident grid any
// cap is slower.
constexpr int kSpillBlocksPerCU = 12;
// Tile order: 16 cells per axis at most, Morton-numbered buckets.
constexpr int kOrderCellsLog = 4;
constexpr int kOrderBuckets = 1 << (3 * kOrderCellsLog);
// Lookahead distance of the tile order, in units of the near range: where a
// unit's centre ray is this far out keys the unit. Grids beyond the Infinity
// Cache key further out (their rays' working sets are what the order has to
// keep apart): on the 1 GiB track 1.5 beat 1.2 by 1.5% and 2.0 by 0.4%;
// on the cache-resident grids 1.2 is within noise of the best (1.0-1.2).
constexpr float kOrderLookahead = 1.2f;
constexpr float kOrderLookaheadSpilled = 1.5f;
// Renders of fewer tiles skip the sort by default: its two launches cost
// ~9 us, more than it saves below ~512 envs of 128x64.
constexpr int64_t kOrderMinTiles = 1 << 16;
// Waves per workgroup of the tiles schedule. A workgroup's slot on the CU is
// freed only when its slowest wave ends, so small workgroups waste fewer
// wave slots on the long-ray tail; two (rather than one) keep the per-
// workgroup LDS axis tables within the CU's LDS at full occupancy on the
// largest grids.
constexpr int kTileWaves = 2;
// Sorted tile-order blocks are dealt to the XCDs in chunks of this many
// workgroups: XCD x takes chunks x, x+8, x+16, ... A chunk keeps one XCD's
// concurrent rays in one part of the map, and interleaving the chunks
// spreads cheap regions (sky) and costly ones (grazing ground) evenly over
// the XCDs, which a contiguous eighth per XCD does not.
constexpr int kXcdChunk = 64;
// A voxel byte offset no ray has sampled: real offsets are multiples of
// the voxel size (2 or 4 bytes).
constexpr uint32_t kNoVoxel = 0xffffffffu;
// Rays per lane by render size (a handle left at rays_per_lane 0): renders
// of fewer tiles than this are latency-bound (few rounds of waves, the
// longest rays' step chains set the time), and one tile per wave halves each
// wave's instructions per step: 16-20% faster at 1-16 envs of 128x64, 5% at
// 256; equal at 512, beyond which two tiles per wave win.
constexpr int64_t kSmallRenderTiles = 1 << 16;

// ---------------------------------------------------------------- errors --
thread_local char g_err[512];

__attribute__((format(printf, 2, 3))) int32_t fail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

}  // namespace

// ---------------------------------------------------------------- handle --
struct SdfrGrid {
    SdfrGridDesc desc;
    int32_t store_dtype;   // SDFR_F32 | SDFR_F16
    int32_t layout;        // SDFR_LAYOUT_*
    int32_t bx, by, bz;    // brick counts (BRICK4), else nx, ny, nz
    void* data;            // device copy
    int64_t bytes;
    uint32_t* counters;    // persistent schedule: tile claim counters + exit counter
    int32_t schedule;      // SDFR_SCHED_*
    int32_t refill_lanes;  // persistent schedule: refill when this many lanes are free
    int32_t rays_per_lane; // tiles: rays each lane marches at once (1, 2; 0 = by render size)
    void* nz_data;         // surf mask grid (int8), same layout as data, or null
    int64_t nz_bytes;
    int device;
    int cus;               // compute units of the device
    int lds_per_cu;        // bytes of LDS per CU
    int32_t tile_order;    // SDFR_ORDER_*: the order the tiles schedule takes tiles in
    int64_t order_min_tiles;  // ... applied to renders of at least this many tiles
    uint32_t* order_hist;  // tile-order bucket counts [kOrderBuckets]: zero between renders
    void* march_events[2]; // caller's hipEvent_t pair around the march launch, or nulls
};

namespace {

// ------------------------------------------------------------ grid access --
// Both layouts have a separable byte offset, off(ix,iy,iz) = X(ix) + Y(iy) +
// Z(iz):
//   LINEAR  [nz][ny][nx]:          X = ix,  Y = iy*nx,  Z = iz*ny*nx
//   BRICK4  [bz][by][bx][4][4][4]: X = (ix>>2)*64 + (ix&3)
//                                  Y = (iy>>2)*bx*64 + (iy&3)*4
//                                  Z = (iz>>2)*by*bx*64 + (iz&3)*16
// (in elements, times the element size). Each workgroup keeps the three
// axis tables in LDS, so a march step forms its gather address with three
// LDS reads and one add instead of integer multiplies. The gather itself goes
// through a buffer descriptor: 32-bit offsets, and an offset past the end of
// the copy reads 0 instead of faulting.
__device__ __forceinline__ uint32_t axis_offset(int i, int nx, int ny, int layout, int bx, int by,
                                                int log_elem) {
    uint32_t e;
    if (i < nx) {
        const uint32_t ix = (uint32_t)i;
        e = layout == SDFR_LAYOUT_LINEAR ? ix : ((ix >> 2) << 6) + (ix & 3u);
    } else if (i < nx + ny) {
        const uint32_t iy = (uint32_t)(i - nx);
        e = layout == SDFR_LAYOUT_LINEAR ? iy * (uint32_t)nx
                                         : (iy >> 2) * (uint32_t)bx * 64u + (iy & 3u) * 4u;
    } else {
        const uint32_t iz = (uint32_t)(i - nx - ny);
        e = layout == SDFR_LAYOUT_LINEAR ? iz * (uint32_t)ny * (uint32_t)nx
                                         : (iz >> 2) * (uint32_t)by * (uint32_t)bx * 64u +
                                               (iz & 3u) * 16u;
    }
    return e << log_elem;
}

template <typename GT>
__device__ __forceinline__ float load_voxel(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
    if constexpr (sizeof(GT) == 2) {
        const unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
        return __half2float(__ushort_as_half(h));
    } else {
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
    }
}

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

// (sin x, cos x) of an fp32 angle, each the fp64 value rounded once.
__device__ __forceinline__ float2 sincos_f32(float x) {
    double sd, cd;
    sincos((double)x, &sd, &cd);
    return make_float2((float)sd, (float)cd);
}

// --------------------------------------------------------------- the args --
struct MarchArgs {
    const void* grid;
    uint32_t grid_bytes;          // size of the device copy (the descriptor's range)
    uint32_t dead_off;            // slots and persistent schedules: gather offset for ended
                                  // rays, past the range (reads 0 without touching memory)
    int nx, ny, nz, bx, by, layout;
    int grid_f16;                 // the copy stores fp16 voxels (else fp32)
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
    int n_envs;
    float2* rt;                   // ray tables, rt_stride float2 per env
    int rt_stride;                // H + W + 4
    void* out; int64_t env_stride;
    int32_t* taps;
    int tiles_x, tiles_per_env;
    int64_t total_tiles;
    int nblocks;
    uint32_t* counters;           // persistent schedule only
    int refill_lanes;
    const void* nzmask;           // surf mask: |n_z|*127 int8 copy, same layout
    uint32_t nz_bytes;
    int32_t* perm;                // tiles schedule: logical unit -> unit, or null
    uint32_t* order_hist;         // tile-order bucket counts [kOrderBuckets] (the handle's:
                                  // zero on entry, zeroed again by the march), or null
    uint16_t* order_key;          // bucket of each sorted unit
    uint32_t* order_rank;         // place of each unit within its bucket
    int order_shift;              // voxel index >> shift = tile-order cell
    float lookahead;              // distance along a unit's centre ray that keys it
    int rpl;                      // this render's rays per lane (tiles) or slots per wave
    int order_unit;               // tiles per sorted unit: one workgroup's, kTileWaves * RPL
    int pack_off;                 // tiles schedule: word offset of the packing lane lists in LDS
    int64_t order_units;          // units the order sorts
    int64_t logical_tiles;        // tile slots the tiles schedule walks: total_tiles, or
                                  // order_units * order_unit under a tile order (a last
                                  // partial unit leaves empty slots)
};

// Block b runs on XCD b % 8; give XCD x the x-th contiguous eighth of the
// logical blocks (a bijection for any block count).
__device__ __forceinline__ int xcd_logical_block(int b, int nblocks) {
    int q = nblocks >> 3, rem = nblocks & 7;
    int x = b & 7, i = b >> 3;
    return x * q + (x < rem ? x : rem) + i;
}

// Block b runs on XCD x = b % 8 as that XCD's i-th block (i = b / 8); give
// it logical block ((i / C) * 8 + x) * C + i % C, so XCD x walks chunks x,
// x+8, x+16, ... of C logical blocks. The blocks beyond the last whole round
// of 8 chunks map to themselves (a bijection for any block count).
__device__ __forceinline__ int xcd_chunked_block(int b, int nblocks, int C) {
    const int full = (nblocks / (8 * C)) * 8 * C;
    if (b >= full) return b;
    const int i = b >> 3, x = b & 7;
    const int k = i / C, o = i - k * C;
    return (k * 8 + x) * C + o;
}

// -------------------------------------------------------------- ray setup --
// The grid value every ray of an env reads at its first step: at t = 0 the
// sample point e + d*0 is the eye itself for every direction (e + (+-0) = e
// up to the sign of a zero, which the index formula maps to the same voxel),
// so the whole env shares one first sample. 0 when there is no grid.
__device__ __forceinline__ float eye_sample(const MarchArgs& a, float ex, float ey, float ez) {
    if (!a.grid) return 0.0f;
    const int ix = (int)__builtin_amdgcn_fmed3f((ex - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
    const int iy = (int)__builtin_amdgcn_fmed3f((ey - a.mny) * a.inv_cell, 0.0f, a.fny1);
    const int iz = (int)__builtin_amdgcn_fmed3f((ez - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
    const int lg = a.grid_f16 ? 1 : 2;
    const uint32_t off = axis_offset(ix, a.nx, a.ny, a.layout, a.bx, a.by, lg) +
                         axis_offset(a.nx + iy, a.nx, a.ny, a.layout, a.bx, a.by, lg) +
                         axis_offset(a.nx + a.ny + iz, a.nx, a.ny, a.layout, a.bx, a.by, lg);
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(a.grid), 0, (int)a.grid_bytes, kRsrcWord3);
    return a.grid_f16 ? load_voxel<__half>(rsrc, off) : load_voxel<float>(rsrc, off);
}

// Eye height of env n: origin z + 12 ducked or 17 standing (vision.py:77-78).
__device__ __forceinline__ float eye_z(const MarchArgs& a, int n) {
    const bool dk = read_ducked(a.ducked, n * a.ducked_stride, a.ducked_dtype);
    return a.origin[n * a.origin_stride + 2] + (dk ? 12.0f : 17.0f);
}

// Ray table of env n, entries (float2):
//   [0, H)       rows:    equiangular (sin, cos) of pitch + poff[r];  pinhole (v[r], 0)
//   [H, H+W)     columns: equiangular (sin, cos) of yaw + yoff[c];    pinhole (u[c], 0)
//   H+W, H+W+1   eye: (x, y), (z, s0) with s0 the grid value at the eye voxel
//   H+W+2, +3    pinhole only: (sin, cos) of the view pitch, of the view yaw
// (vision.py:68-84 kernel setup; :596-624 the CPU path's _dirs_equiangular
// and _dirs_pinhole; :499-529 the offset tables.)
__device__ __forceinline__ float2 table_entry(const MarchArgs& a, int n, int e) {
    const float yr = a.yaw[n * a.yaw_stride] * kD2Rf;
    const float pr = a.pitch[n * a.pitch_stride] * kD2Rf;
    if (e < a.H) {
        if (a.camera == SDFR_CAM_EQUIANGULAR) return sincos_f32(pr + equiangular_offset(e, a.H, a.vfov));
        return make_float2(pinhole_v(e, a.H, a.tan_v), 0.0f);
    }
    e -= a.H;
    if (e < a.W) {
        if (a.camera == SDFR_CAM_EQUIANGULAR) return sincos_f32(yr + equiangular_offset(e, a.W, a.hfov));
        return make_float2(pinhole_u(e, a.W, a.tan_h), 0.0f);
    }
    e -= a.W;
    if (e == 0) return make_float2(a.origin[n * a.origin_stride + 0], a.origin[n * a.origin_stride + 1]);
    if (e == 1) {
        const float ez = eye_z(a, n);
        return make_float2(ez, eye_sample(a, a.origin[n * a.origin_stride + 0],
                                          a.origin[n * a.origin_stride + 1], ez));
    }
    if (a.camera != SDFR_CAM_PINHOLE) return make_float2(0.0f, 0.0f);
    return sincos_f32(e == 2 ? pr : yr);
}

// Unit direction from a ray's row and column entries (and, pinhole, the
// env's view sin/cos pairs).
template <int CAMERA>
__device__ __forceinline__ float3 ray_dir(float2 row, float2 col, float2 pitch_sc, float2 yaw_sc) {
    if constexpr (CAMERA == SDFR_CAM_EQUIANGULAR) {
        // row = (sin p, cos p), col = (sin y, cos y)
        return make_float3(row.y * col.y, row.y * col.x, row.x);
    } else {
        // forward + u*right + v*up, normalised (vision.py:236-246, :614-624);
        // the CPU path's rsqrt is 1/sqrt with two fp32 roundings
        const float v = row.x, u = col.x;
        const float sp = pitch_sc.x, cp = pitch_sc.y, sy = yaw_sc.x, cy = yaw_sc.y;
        const float px = cp * cy + u * sy - v * sp * cy;
        const float py = cp * sy - u * cy - v * sp * sy;
        const float pz = sp + v * cp;
        const float inv = 1.0f / sqrtf(px * px + py * py + pz * pz);
        return make_float3(px * inv, py * inv, pz * inv);
    }
}

// The encoding, vision.py:112-116 / :654-657; t already clamped to range.
// At t <= near the tail is 0.25*(1 - exp(-0)) = 0 exactly, so it is skipped.
__device__ __forceinline__ float encode_depth(float t, float near) {
    if (!(t > near)) return t / near;
    const float lin = near / near;
    const float xe = -(t - near) / 2500.0f;
    const float ed = (float)exp((double)xe);
    return lin + 0.25f * (1.0f - ed);
}

template <int OUT_DTYPE>
__device__ __forceinline__ void store_enc(void* out, int64_t o, float enc) {
    if constexpr (OUT_DTYPE == SDFR_BF16) ((uint16_t*)out)[o] = f32_to_bf16_rne(enc);
    else ((float*)out)[o] = enc;
}

// One march step of a live ray (vision.py:101-111). Returns whether the ray
// is still alive; t advances only if it is.
template <typename GT>
__device__ __forceinline__ bool march_step(const MarchArgs& a, __amdgpu_buffer_rsrc_t rsrc,
                                           const uint32_t* __restrict__ tab, float ex, float ey,
                                           float ez, float dx, float dy, float dz, float& t) {
    const float px = ex + dx * t;
    const float py = ey + dy * t;
    const float pz = ez + dz * t;
    const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
    const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
    const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
    const float sd = load_voxel<GT>(rsrc, tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz]);
    const bool alive = (sd > a.hit_eps) && (t < a.rng);
    if (alive) t = t + fmaxf(sd * 0.9f, a.min_step);
    return alive;
}

template <typename GT, int LAYOUT>
__device__ __forceinline__ void fill_axis_tables(const MarchArgs& a, uint32_t* s_axis) {
    constexpr int kLog = sizeof(GT) == 2 ? 1 : 2;
    const int ntab = a.nx + a.ny + a.nz;
    for (int i = threadIdx.x; i < ntab; i += blockDim.x)
        s_axis[i] = axis_offset(i, a.nx, a.ny, LAYOUT, a.bx, a.by, kLog);
    __syncthreads();
}

// ------------------------------------------------------------- tile order --
// The tiles schedule can take tiles in a spatial order instead of env order.
// Tiles are sorted in units of one workgroup's tiles (kTileWaves * RPL
// consecutive tiles, side by side in one image row of one env, so the waves
// of a workgroup march similar rays and end together); each unit is keyed by
// where its centre ray is after `lookahead` units of distance (1.2 x the
// near range): the cell (of a grid of at most 16^3 cells over the voxel
// grid) holding that point, numbered along a Morton curve. A counting sort by
// key gives the permutation of units; the march then deals chunks of the
// sorted list to the XCDs (xcd_chunked_block), so at any time each XCD's L2
// serves rays that look at one part of the map. Results do not depend on the
// order (every tile is marched exactly as before); it only changes which
// rays share a cache.
//
// The sort is two passes. The ray-setup launch keys the units, counts them
// per bucket in LDS and adds each block's counts to the handle's bucket
// counts with one atomic per bucket, whose return value places the block's
// units of that bucket after those of the blocks before it (each unit's
// rank within its bucket). order_scatter scans the counts and writes each
// unit to its bucket's start plus its rank. The march zeroes the counts
// again, so the next render (or graph replay) starts from zero.
__device__ __forceinline__ uint32_t spread_bits4(uint32_t v) {
    v &= 15u;
    return (v & 1u) | ((v & 2u) << 2) | ((v & 4u) << 4) | ((v & 8u) << 6);
}

// The key of a unit, from its centre ray, in fast fp32 arithmetic (the ray
// tables are written by the same launch); the key only orders the tiles, so
// its precision does not touch the results.
template <int CAMERA>
__device__ __forceinline__ uint32_t tile_order_key(const MarchArgs& a, int64_t unit) {
    // the unit's centre pixel: the left edge of its middle tile, or the
    // centre of a lone last tile
    const int64_t first = unit * a.order_unit;
    const bool whole = first + a.order_unit <= a.total_tiles;
    const int64_t tile = whole ? first + a.order_unit / 2 : first;
    const int n = (int)(tile / a.tiles_per_env);
    const int rem = (int)(tile - (int64_t)n * a.tiles_per_env);
    const int ty = rem / a.tiles_x;
    const int tx = rem - ty * a.tiles_x;
    const int r = min(ty * 8 + 4, a.H - 1), c = min(tx * 8 + (whole ? 0 : 4), a.W - 1);
    const float yr = a.yaw[n * a.yaw_stride] * kD2Rf;
    const float pr = a.pitch[n * a.pitch_stride] * kD2Rf;
    float2 row, col, psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
    if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
        row = make_float2(pinhole_v(r, a.H, a.tan_v), 0.0f);
        col = make_float2(pinhole_u(c, a.W, a.tan_h), 0.0f);
        psc = make_float2(__sinf(pr), __cosf(pr));
        ysc = make_float2(__sinf(yr), __cosf(yr));
    } else {
        const float p = pr + (float)a.vfov * (0.5f - ((float)r + 0.5f) / (float)a.H) * kD2Rf;
        const float y = yr + (float)a.hfov * (0.5f - ((float)c + 0.5f) / (float)a.W) * kD2Rf;
        row = make_float2(__sinf(p), __cosf(p));
        col = make_float2(__sinf(y), __cosf(y));
    }
    const float3 d = ray_dir<CAMERA>(row, col, psc, ysc);
    const float L = a.lookahead;
    const float ex = a.origin[n * a.origin_stride + 0], ey = a.origin[n * a.origin_stride + 1];
    const float ez = eye_z(a, n);
    const int ix = (int)__builtin_amdgcn_fmed3f((ex + d.x * L - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
    const int iy = (int)__builtin_amdgcn_fmed3f((ey + d.y * L - a.mny) * a.inv_cell, 0.0f, a.fny1);
    const int iz = (int)__builtin_amdgcn_fmed3f((ez + d.z * L - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
    return spread_bits4((uint32_t)ix >> a.order_shift) |
           (spread_bits4((uint32_t)iy >> a.order_shift) << 1) |
           (spread_bits4((uint32_t)iz >> a.order_shift) << 2);
}

// Units per sort block (4 per thread).
constexpr int kOrderChunk = 1024;

// ------------------------------------------------------------- ray setup --
// With the tile order on, blocks [0, sort_blocks) key and count a chunk of
// kOrderChunk units each; the blocks after them fill the ray tables, one
// entry per thread. The sort blocks run ~4x longer than a table block, so
// they come first: dispatched last, they started only once the table blocks
// had been dealt out (at 8192 envs 11 us into the launch) and set its end.
template <int CAMERA>
__global__ __launch_bounds__(256) void ray_setup(MarchArgs a, int sort_blocks) {
    if ((int)blockIdx.x >= sort_blocks) {
        const int64_t i = (int64_t)(blockIdx.x - sort_blocks) * blockDim.x + threadIdx.x;
        if (i >= (int64_t)a.n_envs * a.rt_stride) return;
        const int n = (int)(i / a.rt_stride);
        const int e = (int)(i - (int64_t)n * a.rt_stride);
        a.rt[i] = table_entry(a, n, e);
        return;
    }
    constexpr int kPer = kOrderChunk / 256;
    __shared__ uint32_t h[kOrderBuckets];
    for (int i = threadIdx.x; i < kOrderBuckets; i += blockDim.x) h[i] = 0u;
    __syncthreads();
    const int64_t u0 = (int64_t)blockIdx.x * kOrderChunk;
    uint32_t key[kPer], rank[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int64_t u = u0 + threadIdx.x + j * 256;
        key[j] = 0u;
        rank[j] = 0u;
        if (u < a.order_units) {
            key[j] = tile_order_key<CAMERA>(a, u);
            rank[j] = atomicAdd(&h[key[j]], 1u);
        }
    }
    __syncthreads();
    // this block's first place in each bucket
    for (int b = threadIdx.x; b < kOrderBuckets; b += blockDim.x)
        if (h[b]) h[b] = atomicAdd(&a.order_hist[b], h[b]);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const int64_t u = u0 + threadIdx.x + j * 256;
        if (u < a.order_units) {
            a.order_key[u] = (uint16_t)key[j];
            a.order_rank[u] = h[key[j]] + rank[j];
        }
    }
}

// Each block scans the 4096 bucket counts in LDS (bucket b's first slot in
// the sorted list) and writes its chunk's units to their slots.
__global__ __launch_bounds__(256) void order_scatter(MarchArgs a) {
    constexpr int kPer = kOrderChunk / 256;
    constexpr int kBinsPer = kOrderBuckets / 256;
    __shared__ uint32_t start[kOrderBuckets];  // bucket b's first slot
    __shared__ uint32_t wave_sum[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    // exclusive scan of the counts: 16 buckets per thread
    uint32_t v[kBinsPer], sum = 0;
    for (int j = 0; j < kBinsPer; ++j) {
        v[j] = a.order_hist[tid * kBinsPer + j];
        sum += v[j];
    }
    uint32_t inc = sum;
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(inc, off);
        if (lane >= off) inc += o;
    }
    if (lane == 63) wave_sum[wv] = inc;
    __syncthreads();
    uint32_t run = inc - sum;
    for (int w = 0; w < wv; ++w) run += wave_sum[w];
    for (int j = 0; j < kBinsPer; ++j) {
        start[tid * kBinsPer + j] = run;
        run += v[j];
    }
    __syncthreads();
    const int64_t u0 = (int64_t)blockIdx.x * kOrderChunk;
    for (int j = 0; j < kPer; ++j) {
        const int64_t u = u0 + tid + j * 256;
        if (u >= a.order_units) continue;
        const uint32_t pos = start[a.order_key[u] & (kOrderBuckets - 1)] + a.order_rank[u];
        if ((int64_t)pos < a.order_units) a.perm[pos] = (int32_t)u;
    }
}

// Lane shuffles of the tiles schedule's slot packing.
__device__ __forceinline__ int lane_pull(int src_lane, int v) {
    return __builtin_amdgcn_ds_bpermute(src_lane << 2, v);
}
__device__ __forceinline__ float lane_pull(int src_lane, float v) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}
__device__ __forceinline__ uint32_t lane_rank(uint64_t m) {   // set bits of m below this lane
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// ------------------------------------------------------ schedule: tiles --
// Workgroups of kTileWaves waves. Each wave64 marches RPL 8x8 pixel tiles of
// consecutive tile index (so, mostly, neighbouring tiles of one env): lane l
// holds pixel l of every one of them. Per step a lane issues the gathers of
// all its live rays before using any, so RPL independent loads per lane are
// in flight at once. The loop is bound by the texture path (L1 tag lookups
// of divergent gathers) and by vector instruction issue, about equally.
//
// The step counter is wave-uniform and the loop leaves as soon as no ray of
// the wave is alive, which is exact: alive only turns off and a dead ray adds
// 0 to t. Step 0 needs no gather: every ray of an env samples the eye voxel
// first, and the ray-table pass has read that value once per env.
//
// Slot packing (fp16 grids, RPL 2): once the live rays of a wave's two tiles
// fit in 64 lanes, the second tile's live rays move into the first tile's
// ended lanes (ds_bpermute, lane lists in LDS) and the second slot stops
// issuing address math and gathers. A ray's state travels with it, its
// pixel index included, so results land where they belong; rays march
// exactly as before, only their lane changes.
//
// SURF adds the surf-mask channel (vision.py:118-191): after the march the
// voxel under the clamped depth is re-derived with the same index formula
// and the |n_z| grid (int8, |n_z|*127) is read there; the image is then
// interleaved (depth, |n_z|) per pixel, channel fastest (vision.py:558-570).
template <typename GT, int LAYOUT, int OUT_DTYPE, int CAMERA, bool CENSUS, int RPL, bool SURF>
__global__ __launch_bounds__(64 * kTileWaves) void march_tiles(MarchArgs a) {
    extern __shared__ uint32_t s_axis[];
    fill_axis_tables<GT, LAYOUT>(a, s_axis);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (a.order_hist)   // the sort's counts are spent: clear them for the next render
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kOrderBuckets; i += gridDim.x * blockDim.x)
            a.order_hist[i] = 0u;
    const int blk = a.perm ? xcd_chunked_block(blockIdx.x, a.nblocks, kXcdChunk)
                           : xcd_logical_block(blockIdx.x, a.nblocks);
    const int64_t tile0 = ((int64_t)blk * kTileWaves + wave) * RPL;
    if (tile0 >= a.logical_tiles) return;

    // Slot packing (below): on for fp16 grids, where a gather touches half as
    // many lines and vector issue is the tighter bound; on fp32 grids the
    // texture path binds and packing (rays of two tiles in one gather) costs
    // ~3% more L1 tag accesses than the instructions it saves.
    constexpr bool kPack = RPL == 2 && !SURF && sizeof(GT) == 2;
    float ex[RPL], ey[RPL], ez[RPL], dx[RPL], dy[RPL], dz[RPL], t[RPL];
    int env[RPL], pix[RPL];   // env index and r*W + c of each ray (-1: no pixel)
    int taps[RPL];
    bool alive[RPL], valid[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        const int64_t tile = tile0 + j;
        bool tile_ok = tile < a.logical_tiles;
        int64_t tl = tile_ok ? tile : tile0;
        if (a.perm) {
            // logical tile -> (logical unit, place in it) -> sorted unit's tile
            const int64_t ul = tl / a.order_unit;
            const int64_t u = a.perm[ul];
            tl = u * a.order_unit + (tl - ul * a.order_unit);
            if (u < 0 || u >= a.order_units || tl >= a.total_tiles) {   // an empty slot
                tl = 0;
                tile_ok = false;
            }
        }
        const int n = __builtin_amdgcn_readfirstlane((int)(tl / a.tiles_per_env));
        const int rem = (int)(tl - (int64_t)n * a.tiles_per_env);
        const int ty = __builtin_amdgcn_readfirstlane(rem / a.tiles_x);
        const int tx = __builtin_amdgcn_readfirstlane(rem - ty * a.tiles_x);
        const int r = ty * 8 + (lane >> 3);
        const int c = tx * 8 + (lane & 7);
        valid[j] = tile_ok && r < a.H && c < a.W;
        const int rr = min(r, a.H - 1), cc = min(c, a.W - 1);
        const float2* rt = a.rt + (int64_t)n * a.rt_stride;
        const float2 e01 = rt[a.H + a.W], e2 = rt[a.H + a.W + 1];
        float2 psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
        if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
            psc = rt[a.H + a.W + 2];
            ysc = rt[a.H + a.W + 3];
        }
        const float3 d = ray_dir<CAMERA>(rt[rr], rt[a.H + cc], psc, ysc);
        ex[j] = e01.x;
        ey[j] = e01.y;
        ez[j] = e2.x;
        dx[j] = d.x;
        dy[j] = d.y;
        dz[j] = d.z;
        t[j] = 0.0f;
        taps[j] = 0;
        alive[j] = valid[j];
        env[j] = n;
        pix[j] = valid[j] ? rr * a.W + cc : -1;
        // step 0 from the env's shared eye sample (march_step at t = 0:
        // 0 + step is the step exactly)
        if (a.max_steps > 0 && alive[j]) {
            const float s0 = e2.y;
            if constexpr (CENSUS) taps[j] = 1;
            alive[j] = (s0 > a.hit_eps) && (0.0f < a.rng);
            if (alive[j]) t[j] = fmaxf(s0 * 0.9f, a.min_step);
        }
    }
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(a.grid), 0, (int)a.grid_bytes, kRsrcWord3);
    const uint32_t* __restrict__ tab = s_axis;
    // Liveness is kept as one 64-bit lane mask per tile (scalar registers):
    // a new mask is the old one ANDed with the ballots of the two compares,
    // and inverse_ballot turns it back into the per-lane predicate (the exec
    // mask of the address math and gather), so no vector instruction is spent
    // on bookkeeping. A tile whose rays have all ended skips both.
    // offset and value of each ray's most recent gather (a march step that
    // stays in that voxel reads the value again without a gather). Off where
    // slot packing is on: vector issue binds there, and the compare and the
    // kept offset cost more than the gathers they save (~1%).
    constexpr bool kReuse = !kPack;
    uint32_t last_off[RPL];
    float last_sd[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) { last_off[j] = kNoVoxel; last_sd[j] = 0.0f; }
    uint64_t live[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) live[j] = __builtin_amdgcn_ballot_w64(alive[j]);
    for (int k = 1; k < a.max_steps; ++k) {
        uint64_t any = 0;
#pragma unroll
        for (int j = 0; j < RPL; ++j) any |= live[j];
        if (any == 0) break;
        if constexpr (kPack) {
            if (live[0] != 0 && live[1] != 0 && env[0] == env[1] &&
                __builtin_popcountll(live[0]) + __builtin_popcountll(live[1]) <= 64) {
                // both tiles' live rays fit one slot: move slot 1's live rays
                // into slot 0's ended lanes (the k-th live ray of slot 1 to the
                // k-th ended lane of slot 0), and keep each displaced ended
                // ray's result in the slot-1 registers of the lane it came from
                uint32_t* ls = s_axis + a.pack_off + wave * 128;   // lanes with a ray to move
                uint32_t* lf = ls + 64;                            // lanes that take one
                const uint64_t ms = live[1], mf = ~live[0];
                const uint32_t n1 = (uint32_t)__builtin_popcountll(ms);
                const uint32_t rs = lane_rank(ms), rf = lane_rank(mf);
                const bool in_s = __builtin_amdgcn_inverse_ballot_w64(ms);
                const bool in_f = __builtin_amdgcn_inverse_ballot_w64(mf) && rf < n1;
                if (in_s) ls[rs] = (uint32_t)lane;
                if (in_f) lf[rf] = (uint32_t)lane;
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int from = in_f ? (int)ls[rf] : lane;   // slot-1 ray this lane takes
                const int back = in_s ? (int)lf[rs] : lane;   // ended slot-0 ray it keeps
                const float mdx = lane_pull(from, dx[1]), mdy = lane_pull(from, dy[1]);
                const float mdz = lane_pull(from, dz[1]), mt = lane_pull(from, t[1]);
                const int mpix = lane_pull(from, pix[1]);
                const float bt = lane_pull(back, t[0]);
                const int bpix = lane_pull(back, pix[0]);
                int mtaps = 0, btaps = 0;
                if constexpr (CENSUS) {
                    mtaps = lane_pull(from, taps[1]);
                    btaps = lane_pull(back, taps[0]);
                }
                if (in_f) {
                    dx[0] = mdx; dy[0] = mdy; dz[0] = mdz; t[0] = mt; pix[0] = mpix;
                    if constexpr (CENSUS) taps[0] = mtaps;
                }
                if (in_s) {
                    t[1] = bt; pix[1] = bpix;
                    if constexpr (CENSUS) taps[1] = btaps;
                }
                live[0] |= __builtin_amdgcn_ballot_w64(in_f);
                live[1] = 0;
            }
        }
        float sd[RPL];
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            if (__builtin_amdgcn_inverse_ballot_w64(live[j])) {   // ended lanes issue no gather
                const float px = ex[j] + dx[j] * t[j];
                const float py = ey[j] + dy[j] * t[j];
                const float pz = ez[j] + dz[j] * t[j];
                const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
                const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
                const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
                const uint32_t off = tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz];
                // a step that stays in the voxel of the ray's previous sample
                // reuses that value: same voxel, same sample, one line fewer
                // for the texture path
                if constexpr (!kReuse) last_sd[j] = load_voxel<GT>(rsrc, off);
                else if (off != last_off[j]) { last_sd[j] = load_voxel<GT>(rsrc, off); last_off[j] = off; }
            }
            sd[j] = last_sd[j];
        }
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            if constexpr (CENSUS) taps[j] += __builtin_amdgcn_inverse_ballot_w64(live[j]) ? 1 : 0;
            // alive = alive && s > hit_eps && t < range (vision.py:109); an
            // ended lane's bit stays 0 whatever its compares say
            live[j] &= __builtin_amdgcn_ballot_w64(sd[j] > a.hit_eps) &
                       __builtin_amdgcn_ballot_w64(t[j] < a.rng);
            const float tn = t[j] + fmaxf(sd[j] * 0.9f, a.min_step);
            t[j] = __builtin_amdgcn_inverse_ballot_w64(live[j]) ? tn : t[j];
        }
    }
    constexpr int CH = SURF ? 2 : 1;
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        if (pix[j] >= 0) {
            const float tc = fminf(t[j], a.rng);
            const int64_t o = (int64_t)env[j] * a.env_stride + (int64_t)pix[j] * CH;
            store_enc<OUT_DTYPE>(a.out, o, encode_depth(tc, a.near));
            if constexpr (SURF) {
                // the voxel the march stopped in (vision.py:176-187, :658-665)
                constexpr int kLog = sizeof(GT) == 2 ? 1 : 2;
                const float px = ex[j] + dx[j] * tc;
                const float py = ey[j] + dy[j] * tc;
                const float pz = ez[j] + dz[j] * tc;
                const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
                const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
                const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
                const uint32_t off = (tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz]) >> kLog;
                const __amdgpu_buffer_rsrc_t nz_rsrc = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<void*>(a.nzmask), 0, (int)a.nz_bytes, kRsrcWord3);
                const int8_t v = (int8_t)__builtin_amdgcn_raw_buffer_load_b8(nz_rsrc, off, 0, 0);
                store_enc<OUT_DTYPE>(a.out, o + 1, (float)v / 127.0f);
            }
            if constexpr (CENSUS) a.taps[(int64_t)env[j] * a.H * a.W + pix[j]] = taps[j];
        }
    }
}

// ------------------------------------------------- schedule: persistent --
// A grid that fills every CU once. Each wave keeps 64 independent ray slots;
// a slot whose ray has ended is refilled with the next unstarted ray of the
// wave's tile stream, so a wave no longer idles while its slowest ray
// finishes (ray refill, after Aila & Laine 2009). Refills are batched: they
// run when at least refill_lanes slots are free, one ballot and one prefix
// count (mbcnt) hand out the new rays, and the outputs of the rays that ended
// are written in the same batch.
//
// Tile stream: 8 partitions of the tiles (one per XCD: block b runs on XCD
// b % 8), each a contiguous range of envs, claimed one tile at a time with an
// atomic counter; the next claim is issued as soon as a tile is taken, so its
// latency overlaps the march. A wave whose partition is drained moves on to
// the next one. The last wave to leave resets the counters (no other wave
// touches them after that point), so launches on one stream, and graph
// replays, need no clearing in between.
__device__ __forceinline__ uint32_t claim_raw(const MarchArgs& a, int part, int lane) {
    uint32_t got = 0;
    if (lane == 0) got = atomicAdd(&a.counters[part * kCtrStride], 1u);
    return got;
}

template <typename GT, int LAYOUT, int OUT_DTYPE, int CAMERA, bool CENSUS>
__global__ __launch_bounds__(256) void march_persistent(MarchArgs a) {
    extern __shared__ uint32_t s_axis[];
    fill_axis_tables<GT, LAYOUT>(a, s_axis);
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(a.grid), 0, (int)a.grid_bytes, kRsrcWord3);

    int part = (int)((int64_t)xcd_logical_block(blockIdx.x, a.nblocks) * kParts / a.nblocks);
    uint32_t pending = claim_raw(a, part, lane);   // raw claim on `part`, checked when needed
    int tiles_tried = 0;
    bool more = true;     // the tile stream may still have tiles
    int tn = 0, tr0 = 0, tc0 = 0;   // the tile being handed out
    int pos = 64;         // next unstarted ray in it (64 = none left)

    // per-lane ray
    float ex = 0.f, ey = 0.f, ez = 0.f, dx = 0.f, dy = 0.f, dz = 0.f, t = 0.f;
    int k = 0;
    int64_t o = 0;        // output element of the ray
    int32_t pix = 0;      // n*H*W + r*W + c, for the census
    bool has = false;     // the slot holds a ray (running or ended, not yet written)
    bool alive = false;   // ... and it is still marching

    while (true) {
        const int n_free = 64 - (int)__popcll(__ballot(alive));
        if (n_free >= a.refill_lanes || n_free == 64) {
            // write the rays that ended since the last batch
            if (has && !alive) {
                store_enc<OUT_DTYPE>(a.out, o, encode_depth(fminf(t, a.rng), a.near));
                if constexpr (CENSUS) a.taps[pix] = k;
                has = false;
            }
            // hand new rays to the free slots, from at most two tiles
            for (int round = 0; round < 2 && more; ++round) {
                if (pos >= 64) {
                    // take the pending claim, walking on to the next partition when drained
                    int64_t tile = -1;
                    while (true) {
                        const int64_t lo = a.total_tiles * part / kParts;
                        const int64_t hi = a.total_tiles * (part + 1) / kParts;
                        const uint32_t got = __builtin_amdgcn_readfirstlane(pending);
                        if (lo + (int64_t)got < hi) {
                            tile = lo + (int64_t)got;
                            break;
                        }
                        if (++tiles_tried >= kParts) break;
                        part = (part + 1) & (kParts - 1);
                        pending = claim_raw(a, part, lane);
                    }
                    if (tile < 0) {
                        more = false;
                        break;
                    }
                    pending = claim_raw(a, part, lane);   // next claim, in flight meanwhile
                    tn = (int)(tile / a.tiles_per_env);
                    const int rem = (int)(tile - (int64_t)tn * a.tiles_per_env);
                    const int ty = rem / a.tiles_x;
                    tr0 = ty * 8;
                    tc0 = (rem - ty * a.tiles_x) * 8;
                    pos = 0;
                }
                const uint64_t free_mask = __ballot(!has);
                const int n_give = min((int)__popcll(free_mask), 64 - pos);
                if (n_give == 0) break;
                const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(free_mask >> 32),
                                 __builtin_amdgcn_mbcnt_lo((uint32_t)free_mask, 0u));
                if (!has && rank < n_give) {
                    const int q = pos + rank;
                    const int r = tr0 + (q >> 3), c = tc0 + (q & 7);
                    if (r < a.H && c < a.W) {
                        const float2* rt = a.rt + (int64_t)tn * a.rt_stride;
                        const float2 e01 = rt[a.H + a.W], e2 = rt[a.H + a.W + 1];
                        float2 psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
                        if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
                            psc = rt[a.H + a.W + 2];
                            ysc = rt[a.H + a.W + 3];
                        }
                        const float3 d = ray_dir<CAMERA>(rt[r], rt[a.H + c], psc, ysc);
                        dx = d.x;
                        dy = d.y;
                        dz = d.z;
                        ex = e01.x;
                        ey = e01.y;
                        ez = e2.x;
                        o = (int64_t)tn * a.env_stride + (int64_t)r * a.W + c;
                        pix = (tn * a.H + r) * a.W + c;
                        t = 0.0f;
                        k = 0;
                        has = true;
                        alive = a.max_steps > 0;
                    }
                }
                pos += n_give;
            }
            if (!more && __ballot(has) == 0) break;
        }
        if (alive) {
            alive = march_step<GT>(a, rsrc, s_axis, ex, ey, ez, dx, dy, dz, t);
            ++k;
            alive = alive && k < a.max_steps;
        }
    }
    // the last wave out clears the counters for the next launch
    if (lane == 0) {
        const uint32_t total = gridDim.x * (blockDim.x >> 6);
        const uint32_t done = atomicAdd(&a.counters[kParts * kCtrStride], 1u);
        if (done == total - 1) {
            for (int p = 0; p < kParts; ++p) atomicExch(&a.counters[p * kCtrStride], 0u);
            atomicExch(&a.counters[kParts * kCtrStride], 0u);
        }
    }
}

// ------------------------------------------------------ schedule: slots --
// A grid that fills every CU once; each wave marches R independent 8x8 pixel
// tiles ("slots"), one ray per lane per slot. A slot whose 64 rays have all
// ended writes them and takes the wave's next tile, so a wave keeps R
// coherent gathers in flight until its tiles are done: the tiles schedule's
// coherence without its coupling of R tiles to the slowest ray among them.
// Tiles are dealt statically: the waves of XCD x (blocks x, x+8, ...) stride
// through the x-th eighth of the tile range in step, so an XCD works on a
// few consecutive envs at a time; no atomics, no counters.
struct TileSource {
    int next;    // the wave's next tile
    int stride;  // waves sharing the partition
    int end;     // end of the partition
};

__device__ __forceinline__ int take_tile(TileSource& src) {
    if (src.next >= src.end) return -1;
    const int tile = src.next;
    src.next += src.stride;
    return tile;
}

__device__ __forceinline__ float uniform_f(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

template <typename GT, int LAYOUT, int OUT_DTYPE, int CAMERA, bool CENSUS, int R>
__global__ __launch_bounds__(256) void march_slots(MarchArgs a) {
    extern __shared__ uint32_t s_axis[];
    fill_axis_tables<GT, LAYOUT>(a, s_axis);
    const int lane = threadIdx.x & 63;
    const int lr = lane >> 3, lc = lane & 7;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(a.grid), 0, (int)a.grid_bytes, kRsrcWord3);
    const uint32_t* __restrict__ tab = s_axis;
    // this wave's place among the waves of its XCD's partition
    const int total = (int)a.total_tiles;
    TileSource src;
    {
        const int q = a.nblocks >> 3, rem = a.nblocks & 7;
        const int x = (int)(blockIdx.x & 7);
        const int nb = q + (x < rem ? 1 : 0);            // blocks on this partition
        const int lw = (int)(blockIdx.x >> 3) * 4 + (int)(threadIdx.x >> 6);
        const int lo = (int)((int64_t)total * x / kParts);
        src.end = (int)((int64_t)total * (x + 1) / kParts);
        src.next = __builtin_amdgcn_readfirstlane(lo + lw);
        src.stride = nb * 4;
    }

    // per slot: wave-uniform eye, tile and step count (scalar registers),
    // per-lane direction, depth and liveness
    float ex[R], ey[R], ez[R], dx[R], dy[R], dz[R], t[R];
    bool alive[R];
    int tl[R], steps[R], taps[R];
    auto start = [&](int j) {
        tl[j] = take_tile(src);
        if (tl[j] < 0) return;
        const int n = tl[j] / a.tiles_per_env;
        const int rem = tl[j] - n * a.tiles_per_env;
        const int ty = rem / a.tiles_x;
        const int r = ty * 8 + lr, c = (rem - ty * a.tiles_x) * 8 + lc;
        const float2* rt = a.rt + (int64_t)n * a.rt_stride;
        const float2 e01 = rt[a.H + a.W], e2 = rt[a.H + a.W + 1];
        float2 psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
        if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
            psc = rt[a.H + a.W + 2];
            ysc = rt[a.H + a.W + 3];
        }
        const float3 d = ray_dir<CAMERA>(rt[min(r, a.H - 1)], rt[a.H + min(c, a.W - 1)], psc, ysc);
        ex[j] = uniform_f(e01.x);
        ey[j] = uniform_f(e01.y);
        ez[j] = uniform_f(e2.x);
        dx[j] = d.x;
        dy[j] = d.y;
        dz[j] = d.z;
        t[j] = 0.0f;
        taps[j] = 0;
        steps[j] = 0;
        alive[j] = r < a.H && c < a.W && a.max_steps > 0;
    };
    // slot j's rays have all ended: write them
    auto finish = [&](int j) {
        const int n = tl[j] / a.tiles_per_env;
        const int rem = tl[j] - n * a.tiles_per_env;
        const int ty = rem / a.tiles_x;
        const int r = ty * 8 + lr, c = (rem - ty * a.tiles_x) * 8 + lc;
        if (r < a.H && c < a.W) {
            const int pix = r * a.W + c;
            const int64_t o = (int64_t)n * a.env_stride + pix;
            store_enc<OUT_DTYPE>(a.out, o, encode_depth(fminf(t[j], a.rng), a.near));
            if constexpr (CENSUS) a.taps[(int64_t)n * a.H * a.W + pix] = taps[j];
        }
    };
#pragma unroll
    for (int j = 0; j < R; ++j) start(j);
    while (true) {
        bool any_act = false;
#pragma unroll
        for (int j = 0; j < R; ++j) any_act |= tl[j] >= 0;
        if (!any_act) break;
        float sd[R];
#pragma unroll
        for (int j = 0; j < R; ++j) {
            sd[j] = 0.0f;
            if (tl[j] >= 0) {
                const float px = ex[j] + dx[j] * t[j];
                const float py = ey[j] + dy[j] * t[j];
                const float pz = ez[j] + dz[j] * t[j];
                const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
                const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
                const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
                const uint32_t off = alive[j] ? tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz] : a.dead_off;
                sd[j] = load_voxel<GT>(rsrc, off);
            }
        }
#pragma unroll
        for (int j = 0; j < R; ++j) {
            if (tl[j] < 0) continue;
            if (alive[j]) {
                if constexpr (CENSUS) ++taps[j];
                alive[j] = (sd[j] > a.hit_eps) && (t[j] < a.rng);
                if (alive[j]) t[j] = t[j] + fmaxf(sd[j] * 0.9f, a.min_step);
            }
            ++steps[j];
            if (steps[j] >= a.max_steps) alive[j] = false;
            if (!__any(alive[j])) {
                finish(j);
                start(j);
            }
        }
    }
}

// ----------------------------------------------------------- directions --
// One thread per ray: the directions the march casts, (N,H,W,3) f32, from the
// same table entries and the same ray_dir().
template <int CAMERA>
__global__ __launch_bounds__(256) void ray_dirs_kernel(MarchArgs a, float* dirs, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t hw = (int64_t)a.W * a.H;
    const int n = (int)(i / hw);
    const int pix = (int)(i - (int64_t)n * hw);
    const int r = pix / a.W, c = pix - r * a.W;
    float2 psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
    if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
        psc = table_entry(a, n, a.H + a.W + 2);
        ysc = table_entry(a, n, a.H + a.W + 3);
    }
    const float3 d = ray_dir<CAMERA>(table_entry(a, n, r), table_entry(a, n, a.H + c), psc, ysc);
    dirs[3 * i + 0] = d.x;
    dirs[3 * i + 1] = d.y;
    dirs[3 * i + 2] = d.z;
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
    const bool inside = ix < nx && iy < ny && iz < nz;   // padding is never addressed
    const int64_t s = ((int64_t)iz * ny + iy) * nx + ix;
    if constexpr (sizeof(ST) == 1) {
        dst[i] = inside ? src[s] : (DT)0;
    } else {
        float v = 0.0f;
        if (inside) {
            if constexpr (sizeof(ST) == 2) v = __half2float(((const __half*)src)[s]);
            else v = ((const float*)src)[s];
        }
        if constexpr (sizeof(DT) == 2) ((__half*)dst)[i] = __float2half_rn(v);
        else ((float*)dst)[i] = v;
    }
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
size_t axis_lds_bytes(const MarchArgs& a) {
    return sizeof(uint32_t) * (size_t)(a.nx + a.ny + a.nz);
}

// The rays per lane (tiles) or slots per wave (slots) a render of `tiles`
// 8x8 tiles runs with: the handle's setting, or by default 1 for grids
// beyond the Infinity Cache (fewer rays in flight, fewer misses) and for
// small renders, else 2.
int render_rpl(const SdfrGrid* g, int64_t tiles) {
    if (g->rays_per_lane > 0) return g->rays_per_lane;
    return (g->bytes > kCacheResidentBytes || tiles < kSmallRenderTiles) ? 1 : 2;
}

template <typename GT, int LAYOUT, int OUT, int CAMERA, bool CENSUS, bool SURF>
void launch_tiles(MarchArgs& a, const SdfrGrid* g, hipStream_t st) {
    const int rpl = a.rpl;
    size_t lds = axis_lds_bytes(a);
    if (g->bytes > kCacheResidentBytes && g->lds_per_cu > 0)
        lds = max(lds, (size_t)g->lds_per_cu / kSpillBlocksPerCU);   // cap the workgroups per CU
    const int per_block = kTileWaves * rpl;
    a.nblocks = (int)((a.logical_tiles + per_block - 1) / per_block);
    // slot packing (fp16 grids, 2 rays per lane, no surf channel): two
    // 64-entry lane lists per wave after the axis tables
    a.pack_off = (a.nx + a.ny + a.nz + 63) & ~63;
    const bool pack = rpl == 2 && !SURF && sizeof(GT) == 2;
    const size_t lds_pack = pack ? max(lds, sizeof(uint32_t) * ((size_t)a.pack_off + 128 * kTileWaves)) : lds;
    if (rpl == 2)
        march_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, 2, SURF><<<a.nblocks, 64 * kTileWaves, lds_pack, st>>>(a);
    else
        march_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, 1, SURF><<<a.nblocks, 64 * kTileWaves, lds, st>>>(a);
}

// A grid that fills every CU once (never more waves than tiles) for a
// schedule whose waves drain the per-XCD tile stream.
template <typename K>
int persistent_blocks(K kernel, const MarchArgs& a, const SdfrGrid* g, size_t lds, int tiles_per_wave) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), 256,
                                                     lds) != hipSuccess ||
        per_cu <= 0)
        per_cu = 1;
    const int64_t want = (int64_t)per_cu * (g->cus > 0 ? g->cus : 1);
    const int64_t need = (a.total_tiles + 4 * tiles_per_wave - 1) / (4 * tiles_per_wave);
    // at least one block per XCD partition: every partition's tiles need waves
    return (int)(want < need ? (want > 8 ? want : 8) : (need > 8 ? need : 8));
}

template <typename GT, int LAYOUT, int OUT, int CAMERA, bool CENSUS>
void launch_slots(MarchArgs& a, const SdfrGrid* g, size_t lds, hipStream_t st) {
    switch (a.rpl) {
    case 1:
        a.nblocks = persistent_blocks(march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 1>, a, g, lds, 1);
        march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 1><<<a.nblocks, 256, lds, st>>>(a);
        break;
    case 2:
        a.nblocks = persistent_blocks(march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 2>, a, g, lds, 2);
        march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 2><<<a.nblocks, 256, lds, st>>>(a);
        break;
    case 3:
        a.nblocks = persistent_blocks(march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 3>, a, g, lds, 3);
        march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 3><<<a.nblocks, 256, lds, st>>>(a);
        break;
    default:
        a.nblocks = persistent_blocks(march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 4>, a, g, lds, 4);
        march_slots<GT, LAYOUT, OUT, CAMERA, CENSUS, 4><<<a.nblocks, 256, lds, st>>>(a);
        break;
    }
}

template <typename GT, int LAYOUT, int OUT, int CAMERA, bool CENSUS>
void launch_march(MarchArgs& a, const SdfrGrid* g, bool surf, hipStream_t st) {
    if (surf) {
        // the surf-mask variant exists for the equiangular camera only
        // (vision.py:463-467) and always runs the tiles schedule
        if constexpr (CAMERA == SDFR_CAM_EQUIANGULAR) {
            launch_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, true>(a, g, st);
        }
        return;
    }
    if (g->schedule == SDFR_SCHED_TILES) {
        launch_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, false>(a, g, st);
        return;
    }
    const size_t lds = axis_lds_bytes(a);
    if (g->schedule == SDFR_SCHED_SLOTS) {
        launch_slots<GT, LAYOUT, OUT, CAMERA, CENSUS>(a, g, lds, st);
        return;
    }
    // a grid that fills every CU once, never more blocks than the tiles need
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(march_persistent<GT, LAYOUT, OUT, CAMERA, CENSUS>),
            256, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int64_t want = (int64_t)per_cu * (g->cus > 0 ? g->cus : 1);
    const int64_t need = (a.total_tiles + 3) / 4;
    a.nblocks = (int)(want < need ? want : need);
    march_persistent<GT, LAYOUT, OUT, CAMERA, CENSUS><<<a.nblocks, 256, lds, st>>>(a);
}

template <typename GT, int LAYOUT, int OUT>
void dispatch_cam(MarchArgs& a, const SdfrGrid* g, bool census, bool surf, hipStream_t st) {
    if (a.camera == SDFR_CAM_PINHOLE) {
        if (census) launch_march<GT, LAYOUT, OUT, SDFR_CAM_PINHOLE, true>(a, g, surf, st);
        else launch_march<GT, LAYOUT, OUT, SDFR_CAM_PINHOLE, false>(a, g, surf, st);
    } else {
        if (census) launch_march<GT, LAYOUT, OUT, SDFR_CAM_EQUIANGULAR, true>(a, g, surf, st);
        else launch_march<GT, LAYOUT, OUT, SDFR_CAM_EQUIANGULAR, false>(a, g, surf, st);
    }
}

template <typename GT, int LAYOUT>
void dispatch_out(MarchArgs& a, const SdfrGrid* g, int out_dtype, bool census, bool surf,
                  hipStream_t st) {
    if (out_dtype == SDFR_BF16) dispatch_cam<GT, LAYOUT, SDFR_BF16>(a, g, census, surf, st);
    else dispatch_cam<GT, LAYOUT, SDFR_F32>(a, g, census, surf, st);
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
    if ((int64_t)cam->width * cam->height * poses->n_envs > 0x7fffffffLL)
        return fail(-2, "%s: too many rays (%lld, limit 2^31-1)", fn,
                    (long long)cam->width * cam->height * poses->n_envs);
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
    a->n_envs = poses->n_envs;
    a->rt_stride = cam->width + cam->height + 4;
}

// Render workspace: the ray tables, then the tile order's permutation, keys
// and ranks (one per unit, sized for one per tile), each 256-byte aligned.
int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

int64_t ray_table_bytes(int width, int height, int n_envs) {
    return align256((int64_t)n_envs * (width + height + 4) * (int64_t)sizeof(float2));
}

int64_t workspace_bytes(int width, int height, int n_envs) {
    const int64_t tiles = (int64_t)((width + 7) / 8) * ((height + 7) / 8) * n_envs;
    return ray_table_bytes(width, height, n_envs) + align256(tiles * (int64_t)sizeof(int32_t)) +
           align256(tiles * (int64_t)sizeof(uint16_t)) + align256(tiles * (int64_t)sizeof(uint32_t));
}

}  // namespace

// ================================================================ C ABI ==
extern "C" {

SDFR_API int32_t sdfr_abi_version(void) { return SDFR_ABI_VERSION; }

SDFR_API const char* sdfr_last_error(void) { return g_err; }

SDFR_API int64_t sdfr_grid_bytes(const SdfrGrid* grid) { return grid ? grid->bytes : -1; }

SDFR_API int64_t sdfr_workspace_bytes(const SdfrCam* cam, int32_t n_envs) {
    g_err[0] = '\0';
    if (!cam || cam->width <= 0 || cam->height <= 0 || n_envs <= 0)
        return fail(-2, "sdfr_workspace_bytes: need a camera with positive size and n_envs >= 1");
    return workspace_bytes(cam->width, cam->height, n_envs);
}

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
    // The kernels address the copy with 32-bit byte offsets through a buffer
    // descriptor, summed from per-axis tables held in LDS (axis_offset).
    const int64_t elem = store_dtype == SDFR_F16 ? 2 : 4;
    if (count * elem > (int64_t)0xffffffffLL ||
        (int64_t)desc->nx + desc->ny + desc->nz > kMaxAxisEntries) {
        fail(-2, "sdfr_grid_create: grid too large (%d x %d x %d, %lld bytes; limits: 4 GiB and "
             "nx+ny+nz <= %d)", desc->nx, desc->ny, desc->nz, (long long)(count * elem),
             kMaxAxisEntries);
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
    g->bytes = count * elem;
    g->data = nullptr;
    g->counters = nullptr;
    g->nz_data = nullptr;
    g->nz_bytes = 0;
    g->schedule = SDFR_SCHED_TILES;
    g->refill_lanes = 16;
    // two tiles per wave while the grid is cache-resident; one when it spills
    // to HBM, where fewer rays in flight thrash fewer DRAM pages
    g->rays_per_lane = 0;   // by grid and render size
    g->cus = 0;
    g->lds_per_cu = 0;
    g->tile_order = SDFR_ORDER_LOOKAHEAD;
    g->order_min_tiles = kOrderMinTiles;
    g->order_hist = nullptr;
    hipError_t e = hipGetDevice(&g->device);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&g->cus, hipDeviceAttributeMultiprocessorCount, g->device);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&g->lds_per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                                  g->device);

    const int64_t src_bytes = nvox * (src_dtype == SDFR_F16 ? 2 : 4);
    void* staged = nullptr;
    const void* dsrc = src;
    if (e == hipSuccess) e = hipMalloc(&g->data, (size_t)g->bytes);
    if (e == hipSuccess) e = hipMalloc((void**)&g->counters, sizeof(uint32_t) * kCounterWords);
    if (e == hipSuccess) e = hipMemsetAsync(g->counters, 0, sizeof(uint32_t) * kCounterWords, st);
    if (e == hipSuccess) e = hipMalloc((void**)&g->order_hist, sizeof(uint32_t) * kOrderBuckets);
    if (e == hipSuccess) e = hipMemsetAsync(g->order_hist, 0, sizeof(uint32_t) * kOrderBuckets, st);
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
        if (g->counters) (void)hipFree(g->counters);
        if (g->order_hist) (void)hipFree(g->order_hist);
        delete g;
        return nullptr;
    }
    return g;
}

SDFR_API void sdfr_grid_destroy(SdfrGrid* grid) {
    if (!grid) return;
    if (grid->data) (void)hipFree(grid->data);
    if (grid->nz_data) (void)hipFree(grid->nz_data);
    if (grid->counters) (void)hipFree(grid->counters);
    if (grid->order_hist) (void)hipFree(grid->order_hist);
    delete grid;
}

SDFR_API int32_t sdfr_grid_attach_surfnz(SdfrGrid* grid, const void* src, int32_t src_on_device,
                                         void* stream) {
    g_err[0] = '\0';
    if (!grid || !grid->data) return fail(-1, "sdfr_grid_attach_surfnz: null grid handle");
    if (!src) return fail(-1, "sdfr_grid_attach_surfnz: null source");
    hipStream_t st = (hipStream_t)stream;
    const int64_t nvox = (int64_t)grid->desc.nx * grid->desc.ny * grid->desc.nz;
    const int64_t count = grid->layout == SDFR_LAYOUT_BRICK4
                              ? (int64_t)grid->bx * grid->by * grid->bz * 64 : nvox;
    void* dst = nullptr;
    void* staged = nullptr;
    const void* dsrc = src;
    hipError_t e = hipMalloc(&dst, (size_t)count);
    if (e == hipSuccess && !src_on_device) {
        e = hipMalloc(&staged, (size_t)nvox);
        if (e == hipSuccess) e = hipMemcpyAsync(staged, src, (size_t)nvox, hipMemcpyHostToDevice, st);
        dsrc = staged;
    }
    if (e == hipSuccess) e = launch_relayout<int8_t, int8_t>(dsrc, dst, grid, count, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (staged) (void)hipFree(staged);
    if (e != hipSuccess) {
        if (dst) (void)hipFree(dst);
        return fail(-4, "sdfr_grid_attach_surfnz: HIP error %s", hipGetErrorString(e));
    }
    if (grid->nz_data) (void)hipFree(grid->nz_data);
    grid->nz_data = dst;
    grid->nz_bytes = count;
    return 0;
}

SDFR_API int32_t sdfr_grid_set_schedule(SdfrGrid* grid, int32_t schedule, int32_t refill_lanes,
                                        int32_t rays_per_lane) {
    g_err[0] = '\0';
    if (!grid) return fail(-1, "sdfr_grid_set_schedule: null grid handle");
    if (schedule != SDFR_SCHED_PERSISTENT && schedule != SDFR_SCHED_TILES &&
        schedule != SDFR_SCHED_SLOTS)
        return fail(-3, "sdfr_grid_set_schedule: unknown schedule %d", schedule);
    if (refill_lanes < 1 || refill_lanes > 64)
        return fail(-2, "sdfr_grid_set_schedule: refill_lanes must be in 1..64 (got %d)",
                    refill_lanes);
    const int max_rpl = schedule == SDFR_SCHED_SLOTS ? 4 : 2;
    if (rays_per_lane < 0 || rays_per_lane > max_rpl)
        return fail(-2, "sdfr_grid_set_schedule: rays_per_lane must be in 0..%d for this schedule "
                    "(got %d; 0 = by grid and render size)", max_rpl, rays_per_lane);
    grid->schedule = schedule;
    grid->refill_lanes = refill_lanes;
    grid->rays_per_lane = rays_per_lane;
    return 0;
}

SDFR_API int32_t sdfr_render_rays_per_lane(const SdfrGrid* grid, const SdfrCam* cam,
                                           int32_t n_envs) {
    g_err[0] = '\0';
    if (!grid) return fail(-1, "sdfr_render_rays_per_lane: null grid handle");
    if (!cam || cam->width < 1 || cam->height < 1 || n_envs < 1)
        return fail(-2, "sdfr_render_rays_per_lane: need a camera with positive size and n_envs >= 1");
    const int64_t tiles = (int64_t)((cam->width + 7) / 8) * ((cam->height + 7) / 8) * n_envs;
    return render_rpl(grid, tiles);
}

SDFR_API int32_t sdfr_grid_set_march_events(SdfrGrid* grid, void* start, void* stop) {
    g_err[0] = '\0';
    if (!grid) return fail(-1, "sdfr_grid_set_march_events: null grid handle");
    if ((start == nullptr) != (stop == nullptr))
        return fail(-2, "sdfr_grid_set_march_events: give both events or neither");
    grid->march_events[0] = start;
    grid->march_events[1] = stop;
    return 0;
}

SDFR_API int32_t sdfr_grid_set_tile_order(SdfrGrid* grid, int32_t order, int64_t min_tiles) {
    g_err[0] = '\0';
    if (!grid) return fail(-1, "sdfr_grid_set_tile_order: null grid handle");
    if (order != SDFR_ORDER_LAUNCH && order != SDFR_ORDER_LOOKAHEAD)
        return fail(-3, "sdfr_grid_set_tile_order: unknown tile order %d", order);
    grid->tile_order = order;
    grid->order_min_tiles = min_tiles < 0 ? kOrderMinTiles : min_tiles;
    return 0;
}

SDFR_API int32_t sdfr_render(const SdfrGrid* grid, const SdfrCam* cam, const SdfrPoses* poses,
                             const SdfrImage* image, void* workspace, int64_t workspace_size,
                             void* stream) {
    g_err[0] = '\0';
    if (!grid || !grid->data) return fail(-1, "sdfr_render: null grid handle");
    if (!image) return fail(-1, "sdfr_render: null image argument");
    int32_t rc = check_cam_poses("sdfr_render", cam, poses);
    if (rc) return rc;
    if (!image->out) return fail(-1, "sdfr_render: null output pointer");
    if (image->dtype != SDFR_F32 && image->dtype != SDFR_BF16)
        return fail(-3, "sdfr_render: output dtype must be f32 or bf16 (got %d)", image->dtype);
    if (image->channels != 1 && image->channels != 2)
        return fail(-3, "sdfr_render: channels must be 1 or 2 (got %d)", image->channels);
    const bool surf = image->channels == 2;
    if (surf && !grid->nz_data)
        return fail(-1, "sdfr_render: 2 channels need a surf-mask grid (sdfr_grid_attach_surfnz)");
    if (surf && cam->camera != SDFR_CAM_EQUIANGULAR)
        return fail(-3, "sdfr_render: the surf-mask channel has no pinhole kernel");
    if (image->env_stride < (int64_t)cam->width * cam->height * image->channels)
        return fail(-2, "sdfr_render: env_stride %lld is smaller than H*W*channels",
                    (long long)image->env_stride);
    const int64_t need = workspace_bytes(cam->width, cam->height, poses->n_envs);
    if (!workspace || workspace_size < need)
        return fail(-2, "sdfr_render: workspace of %lld bytes needed (got %lld)", (long long)need,
                    (long long)workspace_size);
    if (((uintptr_t)workspace & 7u) != 0)
        return fail(-2, "sdfr_render: workspace must be 8-byte aligned");

    MarchArgs a;
    fill_args(&a, cam, poses);
    a.rt = (float2*)workspace;
    a.grid = grid->data;
    a.grid_bytes = (uint32_t)grid->bytes;
    a.grid_f16 = grid->store_dtype == SDFR_F16;
    // an offset at the end of the range is out of range for a 4-byte read;
    // near 4 GiB fall back to offset 0, an ordinary in-range read
    a.dead_off = grid->bytes <= 0xffffff00ll ? (uint32_t)grid->bytes : 0u;
    a.nx = grid->desc.nx;
    a.ny = grid->desc.ny;
    a.nz = grid->desc.nz;
    a.bx = grid->bx;
    a.by = grid->by;
    a.layout = grid->layout;
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
    a.counters = grid->counters;
    a.refill_lanes = grid->refill_lanes;
    a.nzmask = grid->nz_data;
    a.nz_bytes = (uint32_t)grid->nz_bytes;
    a.tiles_x = (cam->width + 7) / 8;
    a.tiles_per_env = a.tiles_x * ((cam->height + 7) / 8);
    a.total_tiles = (int64_t)a.tiles_per_env * poses->n_envs;
    const int64_t nblocks = (a.total_tiles + kTileWaves - 1) / kTileWaves;
    if (nblocks > 0x7fffffff)
        return fail(-2, "sdfr_render: too many envs (%lld blocks)", (long long)nblocks);
    a.nblocks = (int)nblocks;
    a.perm = nullptr;
    a.order_hist = nullptr;
    a.order_key = nullptr;
    a.order_rank = nullptr;
    a.order_shift = 0;
    a.lookahead = (grid->bytes > kCacheResidentBytes ? kOrderLookaheadSpilled : kOrderLookahead) *
                  cam->near;
    a.rpl = render_rpl(grid, a.total_tiles);
    a.order_unit = kTileWaves * a.rpl;
    a.order_units = (a.total_tiles + a.order_unit - 1) / a.order_unit;
    a.logical_tiles = a.total_tiles;
    if (grid->tile_order == SDFR_ORDER_LOOKAHEAD && (grid->schedule == SDFR_SCHED_TILES || surf) &&
        a.total_tiles >= grid->order_min_tiles) {
        uint8_t* ws = (uint8_t*)workspace + ray_table_bytes(cam->width, cam->height, poses->n_envs);
        a.perm = (int32_t*)ws;
        ws += align256(a.total_tiles * (int64_t)sizeof(int32_t));
        a.order_key = (uint16_t*)ws;
        a.logical_tiles = a.order_units * a.order_unit;
        ws += align256(a.total_tiles * (int64_t)sizeof(uint16_t));
        a.order_rank = (uint32_t*)ws;
        a.order_hist = grid->order_hist;
        const int maxdim = max(a.nx, max(a.ny, a.nz));
        while (((maxdim - 1) >> a.order_shift) >= (1 << kOrderCellsLog)) ++a.order_shift;
    }

    hipStream_t st = (hipStream_t)stream;
    const int64_t entries = (int64_t)poses->n_envs * a.rt_stride;
    const int table_blocks = (int)((entries + 255) / 256);
    const int sort_blocks = a.perm ? (int)((a.order_units + kOrderChunk - 1) / kOrderChunk) : 0;
    if (cam->camera == SDFR_CAM_PINHOLE)
        ray_setup<SDFR_CAM_PINHOLE><<<table_blocks + sort_blocks, 256, 0, st>>>(a, sort_blocks);
    else
        ray_setup<SDFR_CAM_EQUIANGULAR><<<table_blocks + sort_blocks, 256, 0, st>>>(a, sort_blocks);
    if (sort_blocks) order_scatter<<<sort_blocks, 256, 0, st>>>(a);
    const bool census = image->taps != nullptr;
    if (grid->march_events[0] &&
        hipEventRecord((hipEvent_t)grid->march_events[0], st) != hipSuccess)
        return fail(-4, "sdfr_render: recording the march start event failed");
    if (grid->store_dtype == SDFR_F16) {
        if (grid->layout == SDFR_LAYOUT_BRICK4)
            dispatch_out<__half, SDFR_LAYOUT_BRICK4>(a, grid, image->dtype, census, surf, st);
        else
            dispatch_out<__half, SDFR_LAYOUT_LINEAR>(a, grid, image->dtype, census, surf, st);
    } else {
        if (grid->layout == SDFR_LAYOUT_BRICK4)
            dispatch_out<float, SDFR_LAYOUT_BRICK4>(a, grid, image->dtype, census, surf, st);
        else
            dispatch_out<float, SDFR_LAYOUT_LINEAR>(a, grid, image->dtype, census, surf, st);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-4, "sdfr_render: launch failed: %s", hipGetErrorString(e));
    if (grid->march_events[1] &&
        hipEventRecord((hipEvent_t)grid->march_events[1], st) != hipSuccess)
        return fail(-4, "sdfr_render: recording the march stop event failed");
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
    if (cam->camera == SDFR_CAM_PINHOLE)
        ray_dirs_kernel<SDFR_CAM_PINHOLE><<<(int)blocks, 256, 0, (hipStream_t)stream>>>(a, dirs, total);
    else
        ray_dirs_kernel<SDFR_CAM_EQUIANGULAR><<<(int)blocks, 256, 0, (hipStream_t)stream>>>(a, dirs, total);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-4, "sdfr_ray_dirs: launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
