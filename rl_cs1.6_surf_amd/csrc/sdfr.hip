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
// One render is one to three launches on the caller's stream:
//   1. ray_setup: per env, the (sin, cos) of its H row pitch angles and W
//      column yaw angles, and its eye point — all the transcendental work of
//      ray setup, (H+W) fp64 sincos per env instead of two per ray;
//      With the lookahead tile order the same launch also keys the tiles by
//      where they look and counts them into buckets, and order_scatter
//      writes the sorted list (see "tile order"). A small unsorted render
//      (under 8192 tiles, one ray per lane) skips this launch: each march
//      wave builds the table entries of its own tile;
//   2. the march, in one of two schedules with identical results:
//      - tiles (default): launch-scheduled two-wave workgroups, each wave
//        marching RPL 16x4 pixel tiles at once, RPL rays per lane (1 or 2,
//        chosen per render by render_rpl unless the caller fixes it);
//      - persistent: a grid that fills the GPU once; each wave keeps 64 ray
//        slots and refills finished slots with new rays (ray compaction),
//        pulling 16x4 pixel tiles from per-XCD work counters. It keeps every
//        lane busy but mixes rays of different depths in one gather, which
//        costs more cache lines per gather than it saves in idle lanes on
//        the scenes measured so far, so it is not the default.
// Blocks are dealt to the 8 XCDs round-robin by the hardware; they are
// numbered so that each XCD works on a contiguous run of envs (env order), or
// on interleaved chunks of the sorted tile list (lookahead order), keeping
// rays that share grid data in one L2.
//
// Grid storage (the handle's copy): fp32 or fp16 voxels, in 4x4x4 bricks or
// the reference's linear order, or "r16" bricks: per 4x4x4 brick a header
// (fp32 base = the brick's smallest value, fp32 scale = a power of two) and
// 64 uint16 codes, the voxel value being f32(base + code*scale) with
// |value - grid| <= scale/2 plus one fp32 rounding. Two bytes per voxel like
// fp16, but the error is bounded by the brick's own value range (at most
// ~3*sqrt(3)*cell for a distance field: 2^-9 u at 16 u cells) instead of by
// the value's magnitude (fp16: 1 u at 1024-2048 u).

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <type_traits>

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
// cap is slower. A march that reads border voxels from the face copies
// misses less and is faster uncapped (1 GiB f32 grid, 2048 envs: 1.842 ms
// capped at 12, 1.811 uncapped; 512 MiB f16 1.665 / 1.626), so the cap holds
// only without them (f32 2.026 / 2.037, r16 2.704 / 2.834).
constexpr int kSpillBlocksPerCU = 12;
// Tile order: 16 cells per axis at most, Morton-numbered buckets.
constexpr int kOrderCellsLog = 4;
constexpr int kOrderBuckets = 1 << (3 * kOrderCellsLog);
static_assert(kOrderBuckets % 256 == 0, "the sort blocks' 256 threads take 16 buckets each");
// Lookahead distance of the tile order, in units of the near range: where a
// unit's centre ray is this far out keys the unit. Grids beyond the Infinity
// Cache key further out (their rays' working sets are what the order has to
// keep apart): on the 1 GiB track, with its border voxels read from the
// face copies, 3.0 beats 1.5 by 0.9-2.7% at 1024-4096 envs (2.0: 2.6%
// slower); on the cache-resident grids 1.2 is within noise of the best
// (1.0-1.2).
constexpr float kOrderLookahead = 1.2f;
constexpr float kOrderLookaheadSpilled = 3.0f;
// Renders of fewer tiles skip the sort by default: its two launches cost
// ~9 us, more than it saves below ~512 envs of 128x64.
constexpr int64_t kOrderMinTiles = 1 << 16;
// Waves per workgroup of the tiles schedule. A workgroup's slot on the CU is
// freed only when its slowest wave ends, so small workgroups waste fewer
// wave slots on the long-ray tail; two (rather than one) keep the per-
// workgroup LDS axis tables within the CU's LDS at full occupancy on the
// largest grids.
constexpr int kTileWaves = 2;
// A tile is the 64 pixels one wave marches together: 16 columns x 4 rows,
// lane l at (row l / 16, column l % 16). Rays of one image row share a pitch
// and so, over flat ground, similar lengths; a wide tile keeps the wave's
// rays ending together (on the oracle's step counts at ramp_field, 5% fewer
// tile steps than 8x8 tiles and 2% fewer cache lines over the render;
// sparse_grazing 8% / 2%). Tiles are numbered in quads of 2x2 tiles (32x8
// pixels: the upper two side by side, then the lower two), quads row-major
// over the image, so a wave's RPL tiles lie side by side in the same rows
// and a workgroup's tiles form one block of the image.
constexpr int kTileW = 16, kTileH = 4, kTileWLog = 4;
constexpr int kQuadW = 2 * kTileW, kQuadH = 2 * kTileH;
static_assert(kTileW * kTileH == 64 && (1 << kTileWLog) == kTileW, "a tile is one wave's 64 lanes");

// Tiles per env of a width x height image (whole quads).
int64_t tiles_per_env(int width, int height) {
    return (int64_t)((width + kQuadW - 1) / kQuadW) * ((height + kQuadH - 1) / kQuadH) * 4;
}

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
#ifndef SDFR_INLINE_SETUP_TILES
#define SDFR_INLINE_SETUP_TILES (1 << 13)
#endif
constexpr int64_t kInlineSetupTiles = SDFR_INLINE_SETUP_TILES;
// Renders of at least this many tiles (128 envs of 128x64) read border
// voxels from the face copies on grids beyond the Infinity Cache.
constexpr int64_t kFacesMinTiles = 1 << 14;

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
    int32_t store_dtype;   // SDFR_F32 | SDFR_F16 | SDFR_R16
    int32_t layout;        // SDFR_LAYOUT_*
    int32_t bx, by, bz;    // brick counts (BRICK4), else nx, ny, nz
    void* data;            // device copy
    int64_t bytes;         // all of it (r16: codes, padding and brick headers)
    int64_t code_bytes;    // the voxel values (r16: the uint16 codes), from offset 0
    int64_t hdr_off;       // r16: byte offset of the brick headers (float2 per brick), else 0
    int64_t store_bytes;   // the voxel store alone (codes and r16 headers): what the
                           // cache-residence rules look at
    bool has_faces;        // f32/f16 bricks: border faces copied after the bricks
    uint32_t face_off[3];  // byte offset of the z, y and x face pairs (low face first)
    uint32_t face_bytes[3];// bytes of one face of each pair
    int face_lines[2];     // face lines along x (z and y faces) and along y (x faces)
    int32_t border_faces;  // SDFR_FACES_*: when the one-ray march reads them
    uint32_t* counters;    // persistent schedule: tile claim counters + exit counter
    int32_t schedule;      // SDFR_SCHED_*
    int32_t refill_lanes;  // persistent schedule: refill when this many lanes are free
    int32_t rays_per_lane; // tiles: rays each lane marches at once (1, 2; 0 = by render size)
    void* nz_data;         // surf mask grid (int8), same layout as data, or null
    int64_t nz_bytes;
    int device;
    int cus;               // compute units of the device
    int lds_per_cu;        // bytes of LDS per CU
    int lds_per_block;     // largest LDS allocation of one workgroup
    int32_t tile_order;    // SDFR_ORDER_*: the order the tiles schedule takes tiles in
    int64_t order_min_tiles;  // ... applied to renders of at least this many tiles
    uint32_t* order_hist;  // tile-order bucket counts [kOrderBuckets]: zero between renders
    mutable bool hist_dirty;  // a sorted render stopped after counting and before the march
                              // that clears the counts: the next render clears them first
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

// Storage tag of r16 bricks (uint16 codes + per-brick float2 header).
struct R16 {};

template <typename GT>
constexpr int kElemLog = std::is_same<GT, float>::value ? 2 : 1;   // log2 bytes per stored voxel

// Slot packing of the tiles schedule (march_tiles), on for r16 bricks,
// where each sample is up to two gathers (code and brick header) and fewer
// gather instructions pay: ramp_field_r16_bf16's march 2.266 ms with
// packing, 2.365 without, 2.323 with packing and voxel reuse together. On
// fp16 bricks voxel reuse without packing is faster (1.664 against
// 1.712 ms), so fp16 does not pack unless built with SDFR_F16_PACK=1.
#ifndef SDFR_R16_PACK
#define SDFR_R16_PACK 1
#endif
#ifndef SDFR_F16_PACK
#define SDFR_F16_PACK 0
#endif
// r16: a ray keeps the header of the brick it last sampled and gathers only
// the code while it stays in that brick (march 2.266 ms, 2.366 re-reading
// the header at every code gather).
#ifndef SDFR_R16_HDR_REUSE
#define SDFR_R16_HDR_REUSE 1
#endif
template <typename GT>
constexpr bool kPackStore = (std::is_same<GT, __half>::value && SDFR_F16_PACK) ||
                            (std::is_same<GT, R16>::value && SDFR_R16_PACK);

// The record count is the descriptor's unsigned 32-bit byte range; the
// builtin takes it as an int, and the cast keeps its bits, so a copy of up to
// 4 GiB - 1 is addressed whole (offsets are unsigned 32-bit throughout).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, kRsrcWord3);
}

// Reads the voxel at a byte offset of the copy (an offset from the axis
// tables) as fp32. r16: code at `off`, header of its brick at (off / 128) * 8
// (a brick's 64 codes are one 128-byte line); f32(base + code*scale) with the
// product exact (16-bit code, power-of-two scale), so the fma rounds once,
// as the add after an exact multiply does.
template <typename GT>
struct GridReader {
    __amdgpu_buffer_rsrc_t codes, hdr;
    __device__ GridReader(const void* data, uint32_t code_bytes, uint32_t hdr_off, uint32_t hdr_bytes)
        : codes(make_rsrc(data, code_bytes)),
          hdr(make_rsrc((const char*)data + hdr_off, hdr_bytes)) {}
    __device__ __forceinline__ float operator()(uint32_t off) const {
        if constexpr (std::is_same<GT, float>::value) {
            return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(codes, off, 0, 0));
        } else if constexpr (std::is_same<GT, __half>::value) {
            const unsigned short h = __builtin_amdgcn_raw_buffer_load_b16(codes, off, 0, 0);
            return __half2float(__ushort_as_half(h));
        } else {
            const float2 h = header(off);
            return decode(code(off), h);
        }
    }
    // 2-byte stores: the 16-bit code at `off` (fp16 bits, or an r16 code)
    __device__ __forceinline__ uint32_t code(uint32_t off) const {
        return __builtin_amdgcn_raw_buffer_load_b16(codes, off, 0, 0);
    }
    static __device__ __forceinline__ float from_code(uint32_t q) {   // fp16
        return __half2float(__ushort_as_half((unsigned short)q));
    }
    // r16: its brick's (base, scale)
    __device__ __forceinline__ float2 header(uint32_t off) const {
        const auto bs = __builtin_amdgcn_raw_buffer_load_b64(hdr, (off >> 4) & ~7u, 0, 0);
        return make_float2(__uint_as_float(bs[0]), __uint_as_float(bs[1]));
    }
    static __device__ __forceinline__ float decode(uint32_t q, float2 h) {
        return __builtin_fmaf((float)q, h.y, h.x);
    }
};

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
    uint32_t code_bytes;          // bytes of voxel values from `grid` (the codes' descriptor range)
    uint32_t hdr_off, hdr_bytes;  // r16: the brick headers' byte offset and size, else 0
    int nx, ny, nz, bx, by, layout;
    int store;                    // SDFR_F32 | SDFR_F16 | SDFR_R16
    float fnx1, fny1, fnz1;       // n-1 as float: the clamp bound
    float mnx, mny, mnz, inv_cell;
    float smx, smy, smz;          // -mins * inv_cell, exact when pow2_cell
    int pow2_cell;                // inv_cell is a power of two and mins * inv_cell exact
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
    int quads_x, tiles_per_env;   // quads per image row; 4 x quads per env
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
    int inline_setup;             // tiles schedule, small unsorted render: each wave builds its
                                  // tile's ray-table entries itself (no ray-setup launch)
    int faces;                    // one-ray march: border voxels read from the face copies
    int face_alog;                // log2 voxels per row of a face line (3 fp32, 4 fp16)
    int face_lines_x, face_lines_y;
    uint32_t face_off_z, face_off_y, face_off_x;        // low face of each pair
    uint32_t face_bytes_z, face_bytes_y, face_bytes_x;  // one face of each pair
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

// Top-left pixel (row, column) of tile `t` of an env (t < tiles_per_env).
__device__ __forceinline__ int2 tile_corner(const MarchArgs& a, int t) {
    const int quad = t >> 2, q = t & 3;
    const int qy = quad / a.quads_x, qx = quad - qy * a.quads_x;
    return make_int2(qy * kQuadH + (q >> 1) * kTileH, qx * kQuadW + (q & 1) * kTileW);
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
    const int lg = a.store == SDFR_F32 ? 2 : 1;
    const uint32_t off = axis_offset(ix, a.nx, a.ny, a.layout, a.bx, a.by, lg) +
                         axis_offset(a.nx + iy, a.nx, a.ny, a.layout, a.bx, a.by, lg) +
                         axis_offset(a.nx + a.ny + iz, a.nx, a.ny, a.layout, a.bx, a.by, lg);
    if (a.store == SDFR_F32) return GridReader<float>(a.grid, a.code_bytes, 0, 0)(off);
    if (a.store == SDFR_F16) return GridReader<__half>(a.grid, a.code_bytes, 0, 0)(off);
    return GridReader<R16>(a.grid, a.code_bytes, a.hdr_off, a.hdr_bytes)(off);
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

// A sample's coordinate in voxel units along one axis, (p - mins) * inv_cell
// in the reference's two roundings (vision.py:104-106). When inv_cell is a
// power of two the scaling is exact, so round(p - mins) * inv_cell equals
// round((p - mins) * inv_cell), which one fma computes from p and the exact
// product -mins * inv_cell (sm): the same bits, one instruction fewer (any
// result below the normal range truncates to voxel 0 either way).
// A vector instruction reads at most one scalar register, so the fma's two
// per-render constants cannot both stay scalar: inv_cell is handed to the
// loop as a per-lane value (x + 0 * lane, which is x exactly and which the
// compiler must keep in a vector register) and sm stays scalar.
__device__ __forceinline__ float in_vgpr(float x) {
    return x + 0.0f * (float)(threadIdx.x & 63);
}

template <bool POW2>
__device__ __forceinline__ float voxel_coord(float p, float mins, float sm, float inv_cell) {
    if constexpr (POW2) return __builtin_fmaf(p, inv_cell, sm);
    else return (p - mins) * inv_cell;
}

// Border faces. Samples outside the grid clamp to a border voxel
// (vision.py:104-106): on the open synthetic scenes 37-42% of all gathers.
// In 4x4x4 bricks a face's voxels are spread one or two per 64-byte sector
// over the bricks along it, so f32/f16 grids also keep each of the six
// border layers as a 2D copy after the bricks: lines of 128 bytes holding
// 4 rows of 32 bytes (8 fp32 or 16 fp16 voxels) of the face's first axis,
// the lines numbered first-axis-fastest. A voxel on several faces is read
// from the z face, then the y face, then the x face; the copies hold the
// same values, so the choice never changes a result. Face (A, B) of a pair:
// z faces A = ix, B = iy; y faces A = ix, B = iz; x faces A = iy, B = iz.
// Returns the face copy's byte offset of a border voxel, `off` otherwise.
__device__ __forceinline__ uint32_t border_offset(const MarchArgs& a, int ix, int iy, int iz,
                                                  uint32_t off) {
    int A, B, lines;
    uint32_t base;
    if (iz == 0 || iz == a.nz - 1) {
        A = ix; B = iy; lines = a.face_lines_x;
        base = a.face_off_z + (iz != 0 ? a.face_bytes_z : 0u);
    } else if (iy == 0 || iy == a.ny - 1) {
        A = ix; B = iz; lines = a.face_lines_x;
        base = a.face_off_y + (iy != 0 ? a.face_bytes_y : 0u);
    } else if (ix == 0 || ix == a.nx - 1) {
        A = iy; B = iz; lines = a.face_lines_y;
        base = a.face_off_x + (ix != 0 ? a.face_bytes_x : 0u);
    } else {
        return off;
    }
    const int row = (1 << a.face_alog) - 1;
    return base + (uint32_t)(((B >> 2) * lines + (A >> a.face_alog)) * 128 + (B & 3) * 32 +
                             ((A & row) << (5 - a.face_alog)));
}

// One march step of a live ray (vision.py:101-111). Returns whether the ray
// is still alive; t advances only if it is.
template <typename GT>
__device__ __forceinline__ bool march_step(const MarchArgs& a, const GridReader<GT>& rd,
                                           const uint32_t* __restrict__ tab, float ex, float ey,
                                           float ez, float dx, float dy, float dz, float& t) {
    const float px = ex + dx * t;
    const float py = ey + dy * t;
    const float pz = ez + dz * t;
    const int ix = (int)__builtin_amdgcn_fmed3f((px - a.mnx) * a.inv_cell, 0.0f, a.fnx1);
    const int iy = (int)__builtin_amdgcn_fmed3f((py - a.mny) * a.inv_cell, 0.0f, a.fny1);
    const int iz = (int)__builtin_amdgcn_fmed3f((pz - a.mnz) * a.inv_cell, 0.0f, a.fnz1);
    const float sd = rd(tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz]);
    const bool alive = (sd > a.hit_eps) && (t < a.rng);
    if (alive) t = t + fmaxf(sd * 0.9f, a.min_step);
    return alive;
}

template <typename GT, int LAYOUT>
__device__ __forceinline__ void fill_axis_tables(const MarchArgs& a, uint32_t* s_axis) {
    constexpr int kLog = kElemLog<GT>;
    const int ntab = a.nx + a.ny + a.nz;
    for (int i = threadIdx.x; i < ntab; i += blockDim.x)
        s_axis[i] = axis_offset(i, a.nx, a.ny, LAYOUT, a.bx, a.by, kLog);
    __syncthreads();
}

// ------------------------------------------------------------- tile order --
// The tiles schedule can take tiles in a spatial order instead of env order.
// Tiles are sorted in units of one workgroup's tiles (kTileWaves * RPL
// consecutive tiles: the upper or lower half of a quad, or a whole quad, a
// 32-pixel-wide block of one env, so the waves of a workgroup march similar
// rays and end together); each unit is keyed by
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
    // the unit's centre pixel: a unit is two tiles side by side (one quad's
    // upper or lower half) or a whole quad, and starts at a tile with q = 0
    // or 2, so its centre is kTileW right of its first tile's corner and half
    // its height down (units never straddle quads: tiles_per_env is a
    // multiple of 4 and order_unit 2 or 4)
    const int64_t first = unit * a.order_unit;
    const int n = (int)(first / a.tiles_per_env);
    const int2 rc0 = tile_corner(a, (int)(first - (int64_t)n * a.tiles_per_env));
    const int r = min(rc0.x + (a.order_unit == 4 ? kTileH : kTileH / 2), a.H - 1);
    const int c = min(rc0.y + kTileW, a.W - 1);
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
    // this block's first place in each of the thread's 16 buckets: the
    // atomics are independent, so all are issued before any result is
    // awaited (one round trip to memory instead of 16 in a row)
    constexpr int kBinsPer = kOrderBuckets / 256;
    uint32_t cnt[kBinsPer], first[kBinsPer];
#pragma unroll
    for (int j = 0; j < kBinsPer; ++j) cnt[j] = h[threadIdx.x + j * 256];
#pragma unroll
    for (int j = 0; j < kBinsPer; ++j)
        first[j] = cnt[j] ? atomicAdd(&a.order_hist[threadIdx.x + j * 256], cnt[j]) : 0u;
#pragma unroll
    for (int j = 0; j < kBinsPer; ++j) h[threadIdx.x + j * 256] = first[j];
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
// Workgroups of kTileWaves waves. Each wave64 marches RPL 16x4 pixel tiles of
// consecutive tile index (side by side in one env's image): lane l holds
// pixel l of every one of them. Per step a lane issues the gathers of
// all its live rays before using any, so RPL independent loads per lane are
// in flight at once. The loop is bound by the texture path (L1 tag lookups
// of divergent gathers) and by vector instruction issue, about equally.
//
// The step counter is wave-uniform and the loop leaves as soon as no ray of
// the wave is alive, which is exact: alive only turns off and a dead ray adds
// 0 to t. Step 0 needs no gather: every ray of an env samples the eye voxel
// first, and the ray-table pass has read that value once per env.
//
// Slot packing (r16 grids, RPL 2): once the live rays of a wave's two tiles
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

    // Slot packing (below): on for r16 grids, whose samples take up to two
    // gathers; on fp32 grids the texture path binds and packing (rays of
    // two tiles in one gather) costs ~3% more L1 tag accesses than the
    // instructions it saves, and on fp16 grids keeping voxel reuse instead
    // is faster.
    constexpr bool kPack = RPL == 2 && !SURF && kPackStore<GT>;
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
        const int2 rc0 = tile_corner(a, (int)(tl - (int64_t)n * a.tiles_per_env));
        const int r = __builtin_amdgcn_readfirstlane(rc0.x) + (lane >> kTileWLog);
        const int c = __builtin_amdgcn_readfirstlane(rc0.y) + (lane & (kTileW - 1));
        valid[j] = tile_ok && r < a.H && c < a.W;
        const int rr = min(r, a.H - 1), cc = min(c, a.W - 1);
        float2 row, col, e01, e2;
        float2 psc = make_float2(0.f, 0.f), ysc = make_float2(0.f, 0.f);
        if (RPL == 1 && a.inline_setup) {
            // a small render: the wave builds the entries of the env's ray
            // table its tile reads (the values the ray-setup launch would
            // write, by the same function): lanes 0-3 the tile's rows, lanes
            // 4-19 its columns, handed to every lane by ds_bpermute (all 64
            // lanes are active here)
            const int r0 = __builtin_amdgcn_readfirstlane(rc0.x);
            const int c0 = __builtin_amdgcn_readfirstlane(rc0.y);
            float2 mine = make_float2(0.f, 0.f);
            if (lane < kTileH) mine = table_entry(a, n, min(r0 + lane, a.H - 1));
            else if (lane < kTileH + kTileW) mine = table_entry(a, n, a.H + min(c0 + lane - kTileH, a.W - 1));
            const int from_row = lane >> kTileWLog, from_col = kTileH + (lane & (kTileW - 1));
            row = make_float2(lane_pull(from_row, mine.x), lane_pull(from_row, mine.y));
            col = make_float2(lane_pull(from_col, mine.x), lane_pull(from_col, mine.y));
            e01 = table_entry(a, n, a.H + a.W);
            e2 = table_entry(a, n, a.H + a.W + 1);
            if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
                psc = table_entry(a, n, a.H + a.W + 2);
                ysc = table_entry(a, n, a.H + a.W + 3);
            }
        } else {
            const float2* rt = a.rt + (int64_t)n * a.rt_stride;
            row = rt[rr];
            col = rt[a.H + cc];
            e01 = rt[a.H + a.W];
            e2 = rt[a.H + a.W + 1];
            if constexpr (CAMERA == SDFR_CAM_PINHOLE) {
                psc = rt[a.H + a.W + 2];
                ysc = rt[a.H + a.W + 3];
            }
        }
        const float3 d = ray_dir<CAMERA>(row, col, psc, ysc);
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
    const GridReader<GT> rd(a.grid, a.code_bytes, a.hdr_off, a.hdr_bytes);
    const uint32_t* __restrict__ tab = s_axis;
    // Liveness is kept as one 64-bit lane mask per tile (scalar registers):
    // a new mask is the old one ANDed with the ballots of the two compares,
    // and inverse_ballot turns it back into the per-lane predicate (the exec
    // mask of the address math and gather), so no vector instruction is spent
    // on bookkeeping. A tile whose rays have all ended skips both.
    // offset and value of each ray's most recent gather (a march step that
    // stays in that voxel reads the value again without a gather). Off where
    // slot packing is on: a packed slot mixes two tiles' rays, and reuse
    // there measured slower (r16: 2.323 against 2.266 ms).
    constexpr bool kReuse = !kPack;
    constexpr bool kRaw = !std::is_same<GT, float>::value;
    uint32_t last_off[RPL];
    float last_sd[RPL];
    uint32_t last_raw[RPL];   // 2-byte stores: the code of the most recent gather
#pragma unroll
    for (int j = 0; j < RPL; ++j) { last_off[j] = kNoVoxel; last_sd[j] = 0.0f; last_raw[j] = 0u; }
    // r16 with header reuse: the brick (offset / 128) whose header each ray holds
    constexpr bool kHdrReuse = std::is_same<GT, R16>::value && SDFR_R16_HDR_REUSE;
    uint32_t hdr_brick[RPL];
    float2 hdr_val[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) { hdr_brick[j] = kNoVoxel; hdr_val[j] = make_float2(0.f, 0.f); }
    uint64_t live[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) live[j] = __builtin_amdgcn_ballot_w64(alive[j]);
    // Every set-up load lands before the loop, so the loop's waits count
    // only its own gathers. With a set-up load still in flight at the loop's
    // entry the compiler puts a full vmcnt(0) wait inside the loop, before
    // the second tile's address math, and every step then waits for the
    // first tile's gather before issuing the second's: the two gathers of a
    // lane no longer overlap (ramp_field 0.480 -> 0.533 ms).
    __builtin_amdgcn_s_waitcnt(0);
    // The loop, once per form of the voxel index (see voxel_coord: with a
    // power-of-two cell the subtract and the scaling are one fma) and, in the
    // one-ray march, with and without the border face copies.
    const float ic_v = in_vgpr(a.inv_cell);
    auto march = [&](auto pow2_cell, auto border_faces) {
    constexpr bool kPow2 = decltype(pow2_cell)::value;
    constexpr bool kFaces = decltype(border_faces)::value;
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
                    if constexpr (kHdrReuse) hdr_brick[0] = kNoVoxel;   // a moved ray re-reads it
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
                const float ic = kPow2 ? ic_v : a.inv_cell;
                const int ix = (int)__builtin_amdgcn_fmed3f(voxel_coord<kPow2>(px, a.mnx, a.smx, ic), 0.0f, a.fnx1);
                const int iy = (int)__builtin_amdgcn_fmed3f(voxel_coord<kPow2>(py, a.mny, a.smy, ic), 0.0f, a.fny1);
                const int iz = (int)__builtin_amdgcn_fmed3f(voxel_coord<kPow2>(pz, a.mnz, a.smz, ic), 0.0f, a.fnz1);
                const uint32_t off = tab[ix] + tab[a.nx + iy] + tab[a.nx + a.ny + iz];
                // where the value is read: the brick, or for a border voxel
                // of a one-ray march on a grid beyond the Infinity Cache its
                // face copy (see border_offset); `off` stays the voxel's name
                uint32_t at = off;
                if constexpr (kFaces) at = border_offset(a, ix, iy, iz, off);
                // a step that stays in the voxel of the ray's previous sample
                // reuses that value: same voxel, same sample, one line fewer
                // for the texture path
                if constexpr (kRaw) {
                    // 2-byte stores keep the gathered code as it is (and
                    // r16 its brick's header, read only when the ray
                    // enters another brick); it is decoded below
                    if (!kReuse || off != last_off[j]) {
                        last_raw[j] = rd.code(at);
                        if constexpr (std::is_same<GT, R16>::value) {
                            if (!kHdrReuse || (off >> 7) != hdr_brick[j]) {
                                hdr_val[j] = rd.header(off);
                                hdr_brick[j] = off >> 7;
                            }
                        }
                        last_off[j] = off;
                    }
                } else if constexpr (!kReuse) {
                    last_sd[j] = rd(at);
                } else if (off != last_off[j]) {
                    last_sd[j] = rd(at);
                    last_off[j] = off;
                }
            }
        }
        // Decoding a 2-byte code right after its own gather would make the
        // compiler wait for that gather before the next tile's address math,
        // so the gathers of a lane's tiles would not overlap; the codes are
        // decoded once every tile's gathers are issued.
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            if constexpr (kRaw) {
                if constexpr (std::is_same<GT, R16>::value)
                    last_sd[j] = GridReader<GT>::decode(last_raw[j], hdr_val[j]);
                else
                    last_sd[j] = GridReader<GT>::from_code(last_raw[j]);
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
    };
    // each form of the loop is chosen once per wave, not tested per step:
    // a per-step branch on the face flag alone cost small renders 3-6%
    auto with_faces = [&](auto pow2_cell) {
        if constexpr (RPL == 1) {
            if (a.faces) march(pow2_cell, std::true_type{});
            else march(pow2_cell, std::false_type{});
        } else {
            march(pow2_cell, std::false_type{});
        }
    };
    if (a.pow2_cell) with_faces(std::true_type{});
    else with_faces(std::false_type{});
    constexpr int CH = SURF ? 2 : 1;
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        if (pix[j] >= 0) {
            const float tc = fminf(t[j], a.rng);
            const int64_t o = (int64_t)env[j] * a.env_stride + (int64_t)pix[j] * CH;
            store_enc<OUT_DTYPE>(a.out, o, encode_depth(tc, a.near));
            if constexpr (SURF) {
                // the voxel the march stopped in (vision.py:176-187, :658-665)
                constexpr int kLog = kElemLog<GT>;
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
    const GridReader<GT> rd(a.grid, a.code_bytes, a.hdr_off, a.hdr_bytes);

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
                    const int2 rc0 = tile_corner(a, (int)(tile - (int64_t)tn * a.tiles_per_env));
                    tr0 = rc0.x;
                    tc0 = rc0.y;
                    pos = 0;
                }
                const uint64_t free_mask = __ballot(!has);
                const int n_give = min((int)__popcll(free_mask), 64 - pos);
                if (n_give == 0) break;
                const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(free_mask >> 32),
                                 __builtin_amdgcn_mbcnt_lo((uint32_t)free_mask, 0u));
                if (!has && rank < n_give) {
                    const int q = pos + rank;
                    const int r = tr0 + (q >> kTileWLog), c = tc0 + (q & (kTileW - 1));
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
            alive = march_step<GT>(a, rd, s_axis, ex, ey, ez, dx, dy, dz, t);
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

// r16 bricks: one wave per 4x4x4 brick, lane i holding voxel (i&3, (i>>2)&3,
// i>>4) of it. base = the smallest value of the brick's voxels inside the
// grid; scale = 2^e for the smallest e >= -100 with (max - base) <= 65535*2^e
// (e <= 100); code = the value's offset from base in units of scale, rounded
// to nearest even, in [0, 65535]. Offsets and products are formed in fp64
// (exact for the values of a distance field). Padding voxels (never
// addressed) get code 0.
template <typename ST>
__global__ __launch_bounds__(256) void encode_r16(const ST* __restrict__ src, uint16_t* __restrict__ codes,
                                                  float2* __restrict__ hdr, int nx, int ny, int nz, int bx,
                                                  int by, int64_t n_bricks) {
    const int64_t brick = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (brick >= n_bricks) return;   // the whole wave leaves together
    const int lane = threadIdx.x & 63;
    const int64_t bxy = (int64_t)bx * by;
    const int bz_i = (int)(brick / bxy);
    const int by_i = (int)((brick % bxy) / bx);
    const int bx_i = (int)(brick % bx);
    const int ix = bx_i * 4 + (lane & 3), iy = by_i * 4 + ((lane >> 2) & 3), iz = bz_i * 4 + (lane >> 4);
    const bool inside = ix < nx && iy < ny && iz < nz;
    float v = 0.0f;
    if (inside) {
        const int64_t si = ((int64_t)iz * ny + iy) * nx + ix;
        if constexpr (sizeof(ST) == 2) v = __half2float(((const __half*)src)[si]);
        else v = ((const float*)src)[si];
    }
    float lo = inside ? v : INFINITY, hi = inside ? v : -INFINITY;
    for (int m = 1; m < 64; m <<= 1) {
        lo = fminf(lo, __shfl_xor(lo, m));
        hi = fmaxf(hi, __shfl_xor(hi, m));
    }
    const double range = (double)hi - (double)lo;
    int e = -100;
    if (range > 0.0) {
        e = ilogb(range) - 15;               // 2^15 <= range / 2^e < 2^16
        if (ldexp(range, -e) > 65535.0) ++e;
        e = e < -100 ? -100 : (e > 100 ? 100 : e);
    }
    double q = rint(((double)v - (double)lo) * ldexp(1.0, -e));
    q = q >= 0.0 ? (q > 65535.0 ? 65535.0 : q) : 0.0;   // NaN -> 0
    codes[brick * 64 + lane] = inside ? (uint16_t)q : (uint16_t)0;
    if (lane == 0) hdr[brick] = make_float2(lo, ldexpf(1.0f, e));
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

// The copy read back as fp32 [nz][ny][nx], one thread per voxel, through the
// same axis offsets and reader the march uses.
template <typename GT>
__global__ __launch_bounds__(256) void read_grid(MarchArgs a, float* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int ix = (int)(i % a.nx), iy = (int)((i / a.nx) % a.ny), iz = (int)(i / ((int64_t)a.nx * a.ny));
    constexpr int kLog = kElemLog<GT>;
    const uint32_t off = axis_offset(ix, a.nx, a.ny, a.layout, a.bx, a.by, kLog) +
                         axis_offset(a.nx + iy, a.nx, a.ny, a.layout, a.bx, a.by, kLog) +
                         axis_offset(a.nx + a.ny + iz, a.nx, a.ny, a.layout, a.bx, a.by, kLog);
    out[i] = GridReader<GT>(a.grid, a.code_bytes, a.hdr_off, a.hdr_bytes)(off);
}

// --------------------------------------------------------- render dispatch --
size_t axis_lds_bytes(const MarchArgs& a) {
    return sizeof(uint32_t) * (size_t)(a.nx + a.ny + a.nz);
}

// The rays per lane a render of `tiles` tiles runs with: the handle's
// setting, or by default 1 for grids beyond the Infinity Cache (fewer rays in
// flight, fewer misses) and for small renders, else 2.
int render_rpl(const SdfrGrid* g, int64_t tiles) {
    if (g->rays_per_lane > 0) return g->rays_per_lane;
    return (g->store_bytes > kCacheResidentBytes || tiles < kSmallRenderTiles) ? 1 : 2;
}

// One march launch, chosen and sized before anything is enqueued, so that a
// render that cannot launch fails before its ray-setup launch has counted
// tiles into the handle's bucket counts.
struct MarchPlan {
    void (*kernel)(MarchArgs);
    int64_t blocks;
    int threads;
    size_t lds;
};

template <typename GT, int LAYOUT, int OUT, int CAMERA, bool CENSUS, bool SURF>
MarchPlan plan_tiles(MarchArgs& a, const SdfrGrid* g) {
    size_t lds = axis_lds_bytes(a);
    if (g->store_bytes > kCacheResidentBytes && !a.faces && g->lds_per_cu > 0)
        lds = max(lds, (size_t)g->lds_per_cu / kSpillBlocksPerCU);   // cap the workgroups per CU
    const int per_block = kTileWaves * a.rpl;
    const int64_t blocks = (a.logical_tiles + per_block - 1) / per_block;
    // slot packing (2-byte stores, 2 rays per lane, no surf channel): two
    // 64-entry lane lists per wave after the axis tables
    a.pack_off = (a.nx + a.ny + a.nz + 63) & ~63;
    const bool pack = a.rpl == 2 && !SURF && kPackStore<GT>;
    if (pack) lds = max(lds, sizeof(uint32_t) * ((size_t)a.pack_off + 128 * kTileWaves));
    if (a.rpl == 2)
        return {march_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, 2, SURF>, blocks, 64 * kTileWaves, lds};
    return {march_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, 1, SURF>, blocks, 64 * kTileWaves, lds};
}

template <typename GT, int LAYOUT, int OUT, int CAMERA, bool CENSUS>
MarchPlan plan_march(MarchArgs& a, const SdfrGrid* g, bool surf) {
    if (surf) {
        // the surf-mask variant exists for the equiangular camera only
        // (vision.py:463-467) and always runs the tiles schedule
        if constexpr (CAMERA == SDFR_CAM_EQUIANGULAR) return plan_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, true>(a, g);
        return {nullptr, 0, 0, 0};
    }
    if (g->schedule == SDFR_SCHED_TILES) return plan_tiles<GT, LAYOUT, OUT, CAMERA, CENSUS, false>(a, g);
    // persistent: a grid that fills every CU once, never more blocks than the tiles need
    const size_t lds = axis_lds_bytes(a);
    auto k = march_persistent<GT, LAYOUT, OUT, CAMERA, CENSUS>;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(k), 256,
                                                     lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int64_t want = (int64_t)per_cu * (g->cus > 0 ? g->cus : 1);
    const int64_t need = (a.total_tiles + 3) / 4;
    return {k, want < need ? want : need, 256, lds};
}

template <typename GT, int LAYOUT, int OUT>
MarchPlan plan_cam(MarchArgs& a, const SdfrGrid* g, bool census, bool surf) {
    if (a.camera == SDFR_CAM_PINHOLE)
        return census ? plan_march<GT, LAYOUT, OUT, SDFR_CAM_PINHOLE, true>(a, g, surf)
                      : plan_march<GT, LAYOUT, OUT, SDFR_CAM_PINHOLE, false>(a, g, surf);
    return census ? plan_march<GT, LAYOUT, OUT, SDFR_CAM_EQUIANGULAR, true>(a, g, surf)
                  : plan_march<GT, LAYOUT, OUT, SDFR_CAM_EQUIANGULAR, false>(a, g, surf);
}

template <typename GT, int LAYOUT>
MarchPlan plan_out(MarchArgs& a, const SdfrGrid* g, int out_dtype, bool census, bool surf) {
    return out_dtype == SDFR_BF16 ? plan_cam<GT, LAYOUT, SDFR_BF16>(a, g, census, surf)
                                  : plan_cam<GT, LAYOUT, SDFR_F32>(a, g, census, surf);
}

MarchPlan plan_render(MarchArgs& a, const SdfrGrid* g, int out_dtype, bool census, bool surf) {
    if (g->store_dtype == SDFR_R16) return plan_out<R16, SDFR_LAYOUT_BRICK4>(a, g, out_dtype, census, surf);
    if (g->store_dtype == SDFR_F16)
        return g->layout == SDFR_LAYOUT_BRICK4 ? plan_out<__half, SDFR_LAYOUT_BRICK4>(a, g, out_dtype, census, surf)
                                               : plan_out<__half, SDFR_LAYOUT_LINEAR>(a, g, out_dtype, census, surf);
    return g->layout == SDFR_LAYOUT_BRICK4 ? plan_out<float, SDFR_LAYOUT_BRICK4>(a, g, out_dtype, census, surf)
                                           : plan_out<float, SDFR_LAYOUT_LINEAR>(a, g, out_dtype, census, surf);
}

// Clears n words (the tile order's bucket counts) with ordinary vector
// stores: a kernel, not a memset node, so that a caller may capture it.
__global__ __launch_bounds__(256) void clear_words(uint32_t* p, int n) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
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
    const int64_t tiles = tiles_per_env(width, height) * n_envs;
    return ray_table_bytes(width, height, n_envs) + align256(tiles * (int64_t)sizeof(int32_t)) +
           align256(tiles * (int64_t)sizeof(uint16_t)) + align256(tiles * (int64_t)sizeof(uint32_t));
}

// The grid's part of the kernel arguments.
void set_grid_args(MarchArgs* a, const SdfrGrid* grid) {
    a->grid = grid->data;
    a->code_bytes = (uint32_t)grid->code_bytes;
    const bool r16 = grid->store_dtype == SDFR_R16;
    a->hdr_off = r16 ? (uint32_t)grid->hdr_off : 0u;
    a->hdr_bytes = r16 ? (uint32_t)(grid->store_bytes - grid->hdr_off) : 0u;
    a->store = grid->store_dtype;
    a->nx = grid->desc.nx;
    a->ny = grid->desc.ny;
    a->nz = grid->desc.nz;
    a->bx = grid->bx;
    a->by = grid->by;
    a->layout = grid->layout;
    a->fnx1 = (float)(grid->desc.nx - 1);
    a->fny1 = (float)(grid->desc.ny - 1);
    a->fnz1 = (float)(grid->desc.nz - 1);
    a->mnx = grid->desc.mins[0];
    a->mny = grid->desc.mins[1];
    a->mnz = grid->desc.mins[2];
    a->inv_cell = (float)(1.0 / (double)grid->desc.cell);   // Python's 1.0/cell, then fp32
    // -mins * inv_cell for the fma form of the voxel index, used when both
    // that product and inv_cell are exact (inv_cell a power of two)
    int e2 = 0;
    const bool pow2 = frexp((double)a->inv_cell, &e2) == 0.5;
    const double m[3] = {a->mnx, a->mny, a->mnz};
    float sm[3];
    bool exact = pow2;
    for (int i = 0; i < 3; ++i) {
        const double prod = -m[i] * (double)a->inv_cell;
        sm[i] = (float)prod;
        exact = exact && (double)sm[i] == prod && (prod == 0.0 || fabs(prod) >= 0x1p-126);
    }
    a->smx = sm[0];
    a->smy = sm[1];
    a->smz = sm[2];
    a->pow2_cell = exact ? 1 : 0;
}

// The render behind sdfr_render. Everything that can be refused is checked
// and the march launch is planned before the first launch is enqueued. After
// the ray-setup launch has counted tiles into the handle's bucket counts, only
// the march clears them; if a later step fails, the counts are cleared by a
// small kernel, or, if even that cannot be launched, by the next render on the
// handle before its own ray setup (hist_dirty). So a failed render never
// leaves counts that would misplace the next render's tiles.
int32_t render_impl(const char* fn, const SdfrGrid* grid, const SdfrCam* cam, const SdfrPoses* poses,
                    const SdfrImage* image, void* workspace, int64_t workspace_size, void* stream) {
    if (!grid || !grid->data) return fail(-1, "%s: null grid handle", fn);
    if (!image) return fail(-1, "%s: null image argument", fn);
    int32_t rc = check_cam_poses(fn, cam, poses);
    if (rc) return rc;
    if (!image->out) return fail(-1, "%s: null output pointer", fn);
    if (image->dtype != SDFR_F32 && image->dtype != SDFR_BF16)
        return fail(-3, "%s: output dtype must be f32 or bf16 (got %d)", fn, image->dtype);
    if (image->channels != 1 && image->channels != 2)
        return fail(-3, "%s: channels must be 1 or 2 (got %d)", fn, image->channels);
    const bool surf = image->channels == 2;
    if (surf && !grid->nz_data)
        return fail(-1, "%s: 2 channels need a surf-mask grid (sdfr_grid_attach_surfnz)", fn);
    if (surf && cam->camera != SDFR_CAM_EQUIANGULAR)
        return fail(-3, "%s: the surf-mask channel has no pinhole kernel", fn);
    if (image->env_stride < (int64_t)cam->width * cam->height * image->channels)
        return fail(-2, "%s: env_stride %lld is smaller than H*W*channels", fn,
                    (long long)image->env_stride);
    const int64_t need = workspace_bytes(cam->width, cam->height, poses->n_envs);
    if (!workspace || workspace_size < need)
        return fail(-2, "%s: workspace of %lld bytes needed (got %lld)", fn, (long long)need,
                    (long long)workspace_size);
    if (((uintptr_t)workspace & 7u) != 0) return fail(-2, "%s: workspace must be 8-byte aligned", fn);

    MarchArgs a;
    fill_args(&a, cam, poses);
    a.rt = (float2*)workspace;
    set_grid_args(&a, grid);
    a.out = image->out;
    a.env_stride = image->env_stride;
    a.taps = image->taps;
    a.counters = grid->counters;
    a.refill_lanes = grid->refill_lanes;
    a.nzmask = grid->nz_data;
    a.nz_bytes = (uint32_t)grid->nz_bytes;
    a.quads_x = (cam->width + kQuadW - 1) / kQuadW;
    a.tiles_per_env = (int)tiles_per_env(cam->width, cam->height);
    a.total_tiles = (int64_t)a.tiles_per_env * poses->n_envs;
    a.perm = nullptr;
    a.order_hist = nullptr;
    a.order_key = nullptr;
    a.order_rank = nullptr;
    a.order_shift = 0;
    a.lookahead = (grid->store_bytes > kCacheResidentBytes ? kOrderLookaheadSpilled : kOrderLookahead) *
                  cam->near;
    a.rpl = render_rpl(grid, a.total_tiles);
    a.order_unit = kTileWaves * a.rpl;
    a.order_units = (a.total_tiles + a.order_unit - 1) / a.order_unit;
    a.logical_tiles = a.total_tiles;
    a.inline_setup = 0;
    // border face copies: by default for grids beyond the Infinity Cache in
    // renders of at least kFacesMinTiles tiles (the lookup lengthens every
    // step's chain of dependent instructions, which is what a small render's
    // time is made of: winding_track at 1 / 16 / 64 envs 26.4 / 53.6 / 123
    // us without, 35.1 / 62.2 / 127 with; at 256 / 512 envs 342 / 594 without,
    // 315 / 528 with)
    // (only the one-ray march reads them, so the flag says whether this
    // render's march does)
    a.faces = grid->has_faces && a.rpl == 1 &&
              (grid->border_faces == SDFR_FACES_ON ||
               (grid->border_faces == SDFR_FACES_AUTO && grid->store_bytes > kCacheResidentBytes &&
                a.total_tiles >= kFacesMinTiles));
    a.face_alog = grid->store_dtype == SDFR_F32 ? 3 : 4;
    a.face_lines_x = grid->face_lines[0];
    a.face_lines_y = grid->face_lines[1];
    a.face_off_z = grid->face_off[0];
    a.face_off_y = grid->face_off[1];
    a.face_off_x = grid->face_off[2];
    a.face_bytes_z = grid->face_bytes[0];
    a.face_bytes_y = grid->face_bytes[1];
    a.face_bytes_x = grid->face_bytes[2];
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

    // A small unsorted tiles render builds its ray tables inside the march:
    // the 20 table entries a tile reads cost its wave ~1-2 us of fp64 trig,
    // less than the ray-setup launch and the gap before the march (~4 + 3 us;
    // 1-16 envs render 8-13% faster). From ~64 envs on, the trig repeated
    // in every tile costs more than the launch it saves, so larger renders
    // share each env's table among its 128 tiles. Only the one-ray-per-lane
    // march, the default below 65536 tiles, carries the inline path: the
    // fp64 trig doubles a kernel's registers, which the two-ray march of
    // large renders should not pay for.
    if (!a.perm && (grid->schedule == SDFR_SCHED_TILES || surf) && a.total_tiles < kInlineSetupTiles &&
        a.rpl == 1)
        a.inline_setup = 1;

    // plan every launch before enqueueing any
    const bool census = image->taps != nullptr;
    const MarchPlan plan = plan_render(a, grid, image->dtype, census, surf);
    if (!plan.kernel) return fail(-3, "%s: no march kernel for this combination", fn);
    if (plan.blocks < 1 || plan.blocks > 0x7fffffff)
        return fail(-2, "%s: too many envs (%lld march blocks)", fn, (long long)plan.blocks);
    if (grid->lds_per_block > 0 && plan.lds > (size_t)grid->lds_per_block)
        return fail(-2, "%s: the march needs %zu bytes of LDS per workgroup, the device allows %d "
                    "(nx+ny+nz = %d)", fn, plan.lds, grid->lds_per_block, a.nx + a.ny + a.nz);
    a.nblocks = (int)plan.blocks;
    const int64_t entries = (int64_t)poses->n_envs * a.rt_stride;
    const int64_t table_blocks = (entries + 255) / 256;
    const int64_t sort_blocks = a.perm ? (a.order_units + kOrderChunk - 1) / kOrderChunk : 0;
    if (table_blocks + sort_blocks > 0x7fffffff)
        return fail(-2, "%s: too many envs (%lld ray-setup blocks)", fn,
                    (long long)(table_blocks + sort_blocks));

    hipStream_t st = (hipStream_t)stream;
    hipError_t e = hipGetLastError();   // an earlier, unrelated error must not be taken for ours
    (void)e;
    if (grid->hist_dirty) {
        clear_words<<<16, 256, 0, st>>>(grid->order_hist, kOrderBuckets);
        e = hipGetLastError();
        if (e != hipSuccess)
            return fail(-4, "%s: clearing the tile order's counts failed: %s", fn, hipGetErrorString(e));
        grid->hist_dirty = false;
    }
    if (!a.inline_setup) {
        if (cam->camera == SDFR_CAM_PINHOLE)
            ray_setup<SDFR_CAM_PINHOLE><<<(int)(table_blocks + sort_blocks), 256, 0, st>>>(a, (int)sort_blocks);
        else
            ray_setup<SDFR_CAM_EQUIANGULAR><<<(int)(table_blocks + sort_blocks), 256, 0, st>>>(a, (int)sort_blocks);
        e = hipGetLastError();
        if (e != hipSuccess) return fail(-4, "%s: ray setup launch failed: %s", fn, hipGetErrorString(e));
    }
    // from here on a sorted render has counted into order_hist
    auto abandon = [&](const char* what, hipError_t err) -> int32_t {
        if (a.order_hist) {
            clear_words<<<16, 256, 0, st>>>(grid->order_hist, kOrderBuckets);
            grid->hist_dirty = hipGetLastError() != hipSuccess;
        }
        return fail(-4, "%s: %s failed: %s", fn, what, hipGetErrorString(err));
    };
    if (sort_blocks) {
        order_scatter<<<(int)sort_blocks, 256, 0, st>>>(a);
        e = hipGetLastError();
        if (e != hipSuccess) return abandon("tile order launch", e);
    }
    if (grid->march_events[0]) {
        e = hipEventRecord((hipEvent_t)grid->march_events[0], st);
        if (e != hipSuccess) return abandon("recording the march start event", e);
    }
    plan.kernel<<<(int)plan.blocks, plan.threads, plan.lds, st>>>(a);
    e = hipGetLastError();
    if (e != hipSuccess) return abandon("march launch", e);
    if (grid->march_events[1]) {
        e = hipEventRecord((hipEvent_t)grid->march_events[1], st);
        if (e != hipSuccess) return fail(-4, "%s: recording the march stop event failed: %s", fn,
                                         hipGetErrorString(e));
    }
    return 0;
}

// ---------------------------------------------------- allocation-free render --
// sdfr_render_noalloc takes its workspace (ray tables and tile order) from
// this file-scope device array instead of the caller. Each GPU the library
// runs on holds its own copy until the process ends; the host reaches it only
// through the per-device address hipGetSymbolAddress reports (the array's
// name is a host-side stand-in, not a device address). Every call on one GPU
// shares that GPU's copy. Nothing in it needs clearing between calls: the
// ray-setup launch writes every entry a render reads.
constexpr int64_t kScratchBytes = SDFR_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The copy of `scratch` on device `dev` (the current device), looked up once
// per device: by the first sdfr_grid_create on it, which allocates anyway and
// so never runs inside a graph capture, or else by the first allocation-free
// render there.
hipError_t lookup_scratch(int dev, void** out) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

int32_t scratch_for_current_device(const char* fn, const SdfrGrid* grid, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(-4, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
    if (dev != grid->device)
        return fail(-2, "%s: the grid lives on device %d but device %d is current", fn,
                    grid->device, dev);
    if (dev < 0 || dev >= kMaxDevices) return fail(-2, "%s: device %d out of range", fn, dev);
    e = lookup_scratch(dev, out);
    if (e != hipSuccess)
        return fail(-4, "%s: hipGetSymbolAddress(scratch) failed: %s", fn, hipGetErrorString(e));
    return 0;
}

}  // namespace

// ================================================================ C ABI ==
// Copies the six border layers of the source grid into the face copies
// (see border_offset), converting as relayout_grid does, so a face voxel
// holds exactly its brick's value. One thread per face-copy element; rows
// past the face's edge (a line's tail) hold 0 and are never addressed.
template <typename ST, typename DT>
__global__ __launch_bounds__(256) void fill_faces(const ST* __restrict__ src, DT* __restrict__ dst,
                                                  int nx, int ny, int nz, int pair, int high,
                                                  int lines, int64_t count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    constexpr int kRow = 32 / (int)sizeof(DT);                  // voxels per 32-byte row
    constexpr int kLine = 4 * kRow;                             // voxels per 128-byte line
    const int64_t line = i / kLine;
    const int in = (int)(i - line * kLine);
    const int A = (int)(line % lines) * kRow + in % kRow;
    const int B = (int)(line / lines) * 4 + in / kRow;
    int ix, iy, iz, na, nb;
    if (pair == 0) { ix = A; iy = B; iz = high ? nz - 1 : 0; na = nx; nb = ny; }
    else if (pair == 1) { ix = A; iz = B; iy = high ? ny - 1 : 0; na = nx; nb = nz; }
    else { iy = A; iz = B; ix = high ? nx - 1 : 0; na = ny; nb = nz; }
    float v = 0.0f;
    if (A < na && B < nb) {
        const int64_t s = ((int64_t)iz * ny + iy) * nx + ix;
        if constexpr (sizeof(ST) == 2) v = __half2float(((const __half*)src)[s]);
        else v = ((const float*)src)[s];
    }
    if constexpr (sizeof(DT) == 2) ((__half*)dst)[i] = __float2half_rn(v);
    else ((float*)dst)[i] = v;
}

template <typename ST, typename DT>
hipError_t launch_fill_faces(const void* src, SdfrGrid* g, hipStream_t st) {
    for (int f = 0; f < 6; ++f) {
        const int pair = f / 2;
        const int64_t count = g->face_bytes[pair] / (int64_t)sizeof(DT);
        DT* dst = (DT*)((char*)g->data + g->face_off[pair] + (f & 1) * (int64_t)g->face_bytes[pair]);
        fill_faces<ST, DT><<<(int)((count + 255) / 256), 256, 0, st>>>(
            (const ST*)src, dst, g->desc.nx, g->desc.ny, g->desc.nz, pair, f & 1,
            g->face_lines[pair == 2 ? 1 : 0], count);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

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
    if (store_dtype != SDFR_F32 && store_dtype != SDFR_F16 && store_dtype != SDFR_R16) {
        fail(-3, "sdfr_grid_create: store dtype must be f32, f16 or r16 (got %d)", store_dtype);
        copy_err(err, errlen);
        return nullptr;
    }
    if (layout != SDFR_LAYOUT_LINEAR && layout != SDFR_LAYOUT_BRICK4) {
        fail(-3, "sdfr_grid_create: unknown layout %d", layout);
        copy_err(err, errlen);
        return nullptr;
    }
    if (store_dtype == SDFR_R16 && layout != SDFR_LAYOUT_BRICK4) {
        fail(-3, "sdfr_grid_create: the r16 store exists in the brick4 layout only");
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
    const int64_t elem = store_dtype == SDFR_F32 ? 4 : 2;
    const int64_t code_bytes = count * elem;
    const int64_t n_bricks = count / 64;
    const int64_t hdr_off = store_dtype == SDFR_R16 ? align256(code_bytes) : 0;
    const int64_t store_bytes =
        store_dtype == SDFR_R16 ? hdr_off + n_bricks * (int64_t)sizeof(float2) : code_bytes;
    // f32/f16 bricks: the six border layers again, as 2D face copies after
    // the bricks (border_offset), within the same buffer descriptor
    const bool faces = store_dtype != SDFR_R16 && layout == SDFR_LAYOUT_BRICK4;
    const int row = 32 / (int)elem;   // voxels per 32-byte row of a face line
    const int lines_x = (desc->nx + row - 1) / row, lines_y = (desc->ny + row - 1) / row;
    const int64_t face_bytes[3] = {(int64_t)lines_x * ((desc->ny + 3) / 4) * 128,
                                   (int64_t)lines_x * ((desc->nz + 3) / 4) * 128,
                                   (int64_t)lines_y * ((desc->nz + 3) / 4) * 128};
    int64_t face_off[3] = {0, 0, 0};
    int64_t total_bytes = store_bytes;
    if (faces) {
        face_off[0] = align256(store_bytes);
        face_off[1] = face_off[0] + 2 * face_bytes[0];
        face_off[2] = face_off[1] + 2 * face_bytes[1];
        total_bytes = face_off[2] + 2 * face_bytes[2];
    }
    if (total_bytes > (int64_t)0xffffffffLL ||
        (int64_t)desc->nx + desc->ny + desc->nz > kMaxAxisEntries) {
        fail(-2, "sdfr_grid_create: grid too large (%d x %d x %d, %lld bytes; limits: 4 GiB and "
             "nx+ny+nz <= %d)", desc->nx, desc->ny, desc->nz, (long long)total_bytes,
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
    g->bytes = total_bytes;
    g->store_bytes = store_bytes;
    // the buffer descriptor of the voxel reads spans the face copies too
    g->code_bytes = faces ? total_bytes : code_bytes;
    g->hdr_off = hdr_off;
    g->has_faces = faces;
    for (int i = 0; i < 3; ++i) {
        g->face_off[i] = (uint32_t)face_off[i];
        g->face_bytes[i] = faces ? (uint32_t)face_bytes[i] : 0u;
    }
    g->face_lines[0] = lines_x;
    g->face_lines[1] = lines_y;
    g->border_faces = SDFR_FACES_AUTO;
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
    g->hist_dirty = false;
    g->lds_per_block = 0;
    g->march_events[0] = g->march_events[1] = nullptr;
    hipError_t e = hipGetDevice(&g->device);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&g->cus, hipDeviceAttributeMultiprocessorCount, g->device);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&g->lds_per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                                  g->device);
    if (e == hipSuccess)
        e = hipDeviceGetAttribute(&g->lds_per_block, hipDeviceAttributeMaxSharedMemoryPerBlock,
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
    if (e == hipSuccess && store_dtype == SDFR_R16) {
        uint16_t* codes = (uint16_t*)g->data;
        float2* hdr = (float2*)((char*)g->data + hdr_off);
        const int blocks = (int)((n_bricks + 3) / 4);
        if (src_dtype == SDFR_F32)
            encode_r16<float><<<blocks, 256, 0, st>>>((const float*)dsrc, codes, hdr, desc->nx,
                                                      desc->ny, desc->nz, bx, by, n_bricks);
        else
            encode_r16<__half><<<blocks, 256, 0, st>>>((const __half*)dsrc, codes, hdr, desc->nx,
                                                       desc->ny, desc->nz, bx, by, n_bricks);
        e = hipGetLastError();
    } else if (e == hipSuccess) {
        if (src_dtype == SDFR_F32 && store_dtype == SDFR_F32)
            e = launch_relayout<float, float>(dsrc, g->data, g, count, st);
        else if (src_dtype == SDFR_F32)
            e = launch_relayout<float, __half>(dsrc, g->data, g, count, st);
        else if (store_dtype == SDFR_F32)
            e = launch_relayout<__half, float>(dsrc, g->data, g, count, st);
        else
            e = launch_relayout<__half, __half>(dsrc, g->data, g, count, st);
    }
    if (e == hipSuccess && faces) {
        if (src_dtype == SDFR_F32 && store_dtype == SDFR_F32)
            e = launch_fill_faces<float, float>(dsrc, g, st);
        else if (src_dtype == SDFR_F32)
            e = launch_fill_faces<float, __half>(dsrc, g, st);
        else if (store_dtype == SDFR_F32)
            e = launch_fill_faces<__half, float>(dsrc, g, st);
        else
            e = launch_fill_faces<__half, __half>(dsrc, g, st);
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
    // the allocation-free render's scratch on this device: looked up here,
    // outside any capture; a failure is reported by that render's own lookup
    if (g->device >= 0 && g->device < kMaxDevices) {
        void* p = nullptr;
        (void)lookup_scratch(g->device, &p);
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
    if (schedule != SDFR_SCHED_PERSISTENT && schedule != SDFR_SCHED_TILES)
        return fail(-3, "sdfr_grid_set_schedule: unknown schedule %d", schedule);
    if (refill_lanes < 1 || refill_lanes > 64)
        return fail(-2, "sdfr_grid_set_schedule: refill_lanes must be in 1..64 (got %d)",
                    refill_lanes);
    if (rays_per_lane < 0 || rays_per_lane > 2)
        return fail(-2, "sdfr_grid_set_schedule: rays_per_lane must be in 0..2 "
                    "(got %d; 0 = by grid and render size)", rays_per_lane);
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
    return render_rpl(grid, tiles_per_env(cam->width, cam->height) * n_envs);
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

SDFR_API int32_t sdfr_grid_set_border_faces(SdfrGrid* grid, int32_t mode) {
    g_err[0] = '\0';
    if (!grid) return fail(-1, "sdfr_grid_set_border_faces: null grid handle");
    if (mode != SDFR_FACES_AUTO && mode != SDFR_FACES_ON && mode != SDFR_FACES_OFF)
        return fail(-2, "sdfr_grid_set_border_faces: unknown mode %d", mode);
    if (mode == SDFR_FACES_ON && !grid->has_faces)
        return fail(-3, "sdfr_grid_set_border_faces: this grid keeps no face copies (they exist "
                    "for f32 and f16 bricks)");
    grid->border_faces = mode;
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
    return render_impl("sdfr_render", grid, cam, poses, image, workspace, workspace_size, stream);
}

SDFR_API int32_t sdfr_render_noalloc(const SdfrGrid* grid, const SdfrCam* cam,
                                     const SdfrPoses* poses, const SdfrImage* image,
                                     void* stream) {
    g_err[0] = '\0';
    const char* fn = "sdfr_render_noalloc";
    if (!grid || !grid->data) return fail(-1, "%s: null grid handle", fn);
    int32_t rc = check_cam_poses(fn, cam, poses);
    if (rc) return rc;
    const int64_t need = workspace_bytes(cam->width, cam->height, poses->n_envs);
    if (need > kScratchBytes)
        return fail(-2, "%s: %d envs of %dx%d need %lld bytes of workspace; the static scratch "
                    "holds %lld (use sdfr_render with a workspace)", fn, poses->n_envs,
                    cam->width, cam->height, (long long)need, (long long)kScratchBytes);
    void* ws = nullptr;
    rc = scratch_for_current_device(fn, grid, &ws);
    if (rc) return rc;
    return render_impl(fn, grid, cam, poses, image, ws, kScratchBytes, stream);
}

SDFR_API int32_t sdfr_grid_read(const SdfrGrid* grid, float* out, void* stream) {
    g_err[0] = '\0';
    if (!grid || !grid->data) return fail(-1, "sdfr_grid_read: null grid handle");
    if (!out) return fail(-1, "sdfr_grid_read: null output pointer");
    MarchArgs a;
    memset(&a, 0, sizeof a);
    set_grid_args(&a, grid);
    const int64_t n = (int64_t)a.nx * a.ny * a.nz;
    const int64_t blocks = (n + 255) / 256;
    if (blocks > 0x7fffffff) return fail(-2, "sdfr_grid_read: grid too large");
    hipStream_t st = (hipStream_t)stream;
    if (grid->store_dtype == SDFR_R16)
        read_grid<R16><<<(int)blocks, 256, 0, st>>>(a, out, n);
    else if (grid->store_dtype == SDFR_F16)
        read_grid<__half><<<(int)blocks, 256, 0, st>>>(a, out, n);
    else
        read_grid<float><<<(int)blocks, 256, 0, st>>>(a, out, n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(-4, "sdfr_grid_read: launch failed: %s", hipGetErrorString(e));
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
