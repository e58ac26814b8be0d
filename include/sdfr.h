/* sdfr.h — C ABI of the MI355X SDF depth renderer (libsdfr.so).
 *
 * Replaces the per-tick render of the reference's GPU lidar,
 * python/surfgym/vision.py (GpuLidar.__init__ :457-529, GpuLidar.render
 * :542-550, _render_triton :552-594, _march_kernel :59-116). The reference has
 * no C ABI for this path: its Python class launches a Triton JIT kernel. This
 * header is the boundary a ctypes binding (python/surfgym/core.py style:
 * explicit argtypes, ABI-version refusal) loads instead.
 *
 * Conventions follow the reference's own C ABI, src/surfcore.h:
 *   - every array is caller-allocated; device arrays are plain device pointers
 *     (e.g. torch tensor data_ptr()), host structs are passed by pointer;
 *   - creation returns NULL and writes a message into err/errlen
 *     (surfcore.h:156-157); calls return int32 0 = ok, < 0 = error
 *     (surfcore.h:162-168) and sdfr_last_error() says why;
 *   - sdfr_abi_version() is checked by the binding before any other call
 *     (surfcore.h:61-64, core.py:444-448);
 *   - one caller at a time per handle (surfcore.h:4-5).
 *
 * Work is enqueued on the caller's HIP stream (hipStream_t passed as void*,
 * NULL = legacy default stream) and never synchronises the host, so renders
 * order with the caller's other work and can be captured into a hipGraph.
 */
#ifndef SDFR_H
#define SDFR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SDFR_API __attribute__((visibility("default")))

/* Bumped on every struct or semantic change; the binding refuses a library
 * reporting another value. */
#define SDFR_ABI_VERSION 13

/* Element types of caller arrays. */
enum {
    SDFR_F32 = 0,
    SDFR_F16 = 1,
    SDFR_BF16 = 2,
    SDFR_I32 = 3,
    SDFR_I64 = 4,
    SDFR_U8 = 5,   /* also torch.bool */
    SDFR_F64 = 6,
    SDFR_U16 = 7,  /* goal-field grids */
    SDFR_R16 = 8   /* grid store only: 4x4x4 bricks of uint16 codes, each brick with an fp32
                      base (its smallest value) and an fp32 power-of-two scale; a voxel reads
                      f32(base + code*scale), within scale/2 (plus one fp32 rounding) of the
                      source value; scale <= 2^-9 u for a distance field at 16 u cells */
};

/* Device layout of the handle's private copy of the grid. */
enum {
    SDFR_LAYOUT_LINEAR = 0, /* [nz][ny][nx], the reference's sdf_flat order (vision.py:476-480) */
    SDFR_LAYOUT_BRICK4 = 1  /* 4x4x4-voxel bricks, brick-linear, x-fastest inside a brick */
};

/* Camera models (GpuLidar(pinhole=...), vision.py:484-529). */
enum {
    SDFR_CAM_EQUIANGULAR = 0, /* yoff/poff angles added to yaw/pitch (vision.py:502-509) */
    SDFR_CAM_PINHOLE = 1      /* tangent-plane grid, normalised (vision.py:510-529) */
};

/* Work schedules of sdfr_render (both give identical results). */
enum {
    SDFR_SCHED_PERSISTENT = 0, /* persistent waves refilling ended rays' lanes */
    SDFR_SCHED_TILES = 1       /* default: launch-scheduled waves of 16x4 pixel tiles */
};

/* The order in which the tiles schedule takes 16x4 pixel tiles. */
enum {
    SDFR_ORDER_LAUNCH = 0,    /* env by env, as the batch is laid out */
    SDFR_ORDER_LOOKAHEAD = 1  /* default: sorted by where each tile's centre ray is 1.2 x near
                                 units out (Morton order of coarse cells), so each XCD's L2
                                 serves rays looking at one part of the map; applied to
                                 renders of at least min_tiles tiles */
};

/* When the one-ray march reads border voxels from the grid's face copies
 * (f32/f16 bricks keep each of the six border layers again as a 2D copy). */
enum {
    SDFR_FACES_AUTO = 0,  /* default: for grids beyond the Infinity Cache (above 192 MiB) in
                             renders of at least 16384 tiles (128 envs of 128x64) */
    SDFR_FACES_ON = 1,    /* whenever the march runs one ray per lane */
    SDFR_FACES_OFF = 2    /* never */
};

/* Grid geometry: the reference's single grid definition, grid_dims()
 * (vision.py:310-322). Voxel (ix,iy,iz) is sampled at mins + (i+0.5)*cell
 * (env.c:680-682). Values are unsigned distances in map units, 0 in solid. */
typedef struct SdfrGridDesc {
    int32_t nx, ny, nz;
    float mins[3];
    float cell;
} SdfrGridDesc;

/* One sensor configuration: the GpuLidar constructor arguments that reach
 * the march (vision.py:457-509, 99-116). hit_eps and min_step are explicit so
 * callers can pass the reference's 0.6*cell and 0.3*cell (vision.py:87-88) or
 * another epsilon. near == range reproduces the legacy t/range encoding. */
typedef struct SdfrCam {
    int32_t width, height;  /* W, H: pixels per image row / column */
    double hfov_deg;        /* equiangular: horizontal field of view (120) */
    double vfov_deg;        /* equiangular: vertical field of view (90) */
    double tan_half_h;      /* pinhole: tan(hfov/2) as the host computes it (vision.py:517) */
    double tan_half_v;      /* pinhole: tan(vfov/2) (vision.py:518) */
    float range;            /* trace range and clamp (range_units) */
    float near;             /* linear part of the encoding (near_range) */
    float hit_eps;          /* stop when the sampled distance <= hit_eps */
    float min_step;         /* smallest step, max(0.9*d, min_step) */
    int32_t max_steps;      /* loop trip bound */
    int32_t camera;         /* SDFR_CAM_* */
} SdfrCam;

/* Per-env pose inputs (the render() arguments, vision.py:542-550) and the
 * output image. All pointers are device pointers; strides are in elements
 * so strided torch views (the trainer passes columns of an (N,6) tensor,
 * train_fast.py:1757) need no copy. */
typedef struct SdfrPoses {
    const float* origin;     /* (N,3) f32, element (n,a) at origin[n*origin_stride + a] */
    int64_t origin_stride;
    const float* yaw_deg;    /* (N,) f32 degrees */
    int64_t yaw_stride;
    const float* pitch_deg;  /* (N,) f32 degrees */
    int64_t pitch_stride;
    const void* ducked;      /* (N,) any SDFR_* numeric type, nonzero = ducked */
    int64_t ducked_stride;
    int32_t ducked_dtype;
    int32_t n_envs;          /* N >= 1 */
} SdfrPoses;

typedef struct SdfrImage {
    void* out;               /* image of env n at out + n*env_stride elements: row-major HxW,
                                or HxWx2 interleaved (depth, |n_z|) when channels == 2 */
    int64_t env_stride;      /* elements between envs (H*W*channels for a dense tensor) */
    int32_t dtype;           /* SDFR_F32 or SDFR_BF16 */
    int32_t channels;        /* 1 = depth; 2 = depth + surf mask (vision.py:118-191, 558-570) */
    int32_t* taps;           /* optional per-ray census, NULL = off: grid loads issued for the ray,
                                dense (N,H,W) int32 (tools/bench_lidar.py:45-88 counts the same loop) */
} SdfrImage;

typedef struct SdfrGrid SdfrGrid;

SDFR_API int32_t sdfr_abi_version(void);

/* Builds the handle's device copy of a grid. `src` holds nz*ny*nx values of
 * `src_dtype` (SDFR_F32 or SDFR_F16) in [nz][ny][nx] order; src_on_device
 * says whether it is a device pointer (a torch tensor) or host memory.
 * `store_dtype` (SDFR_F32; SDFR_F16, as the reference stores it,
 * vision.py:476-477, rounding to nearest even; or SDFR_R16, brick4 layout
 * only) and `layout` (SDFR_LAYOUT_*) pick the device copy. Replaces the
 * grid upload of GpuLidar.__init__ (vision.py:473-480). The copy is complete when the stream reaches it;
 * the source may be freed after that. NULL + message in err on failure. */
SDFR_API SdfrGrid* sdfr_grid_create(const SdfrGridDesc* desc, const void* src,
                                    int32_t src_dtype, int32_t src_on_device,
                                    int32_t store_dtype, int32_t layout,
                                    void* stream, char* err, int32_t errlen);

SDFR_API void sdfr_grid_destroy(SdfrGrid* grid);

/* Attaches the surf-mask grid to a handle: nz*ny*nx int8 values |n_z|*127
 * in [nz][ny][nx] order, on exactly the SDF's grid (surfmask.py:193-201),
 * re-laid out like the SDF copy. Needed for renders with channels == 2.
 * Replaces the snz_flat upload of GpuLidar.__init__ (vision.py:489-497).
 * Synchronous; 0 or < 0. */
SDFR_API int32_t sdfr_grid_attach_surfnz(SdfrGrid* grid, const void* src, int32_t src_on_device,
                                         void* stream);

/* Chooses how sdfr_render schedules rays on this handle: `schedule` is an
 * SDFR_SCHED_* value (default SDFR_SCHED_TILES); `refill_lanes` (1..64,
 * default 16) is the number of free lanes at which a persistent wave takes
 * new rays; `rays_per_lane` is how many tiles a wave of the tiles schedule
 * marches at once: 1 or 2, or 0 (the default) to let each render choose: 1
 * for grids above 192 MiB and for renders of fewer than 65536 tiles (512
 * envs of 128x64), else 2.
 * Surf-mask renders always use the tiles schedule. Results do not depend
 * on any of them. Synchronous; 0 or < 0. No reference counterpart: the
 * Triton launch has one fixed shape (vision.py:48-54; tools/proto_march.py
 * sweeps it). */
SDFR_API int32_t sdfr_grid_set_schedule(SdfrGrid* grid, int32_t schedule, int32_t refill_lanes,
                                        int32_t rays_per_lane);

/* The rays per lane a render of `n_envs` images of `cam` would run with on
 * this handle (tiles schedule and surf-mask renders); < 0 on bad arguments.
 * No reference counterpart. */
SDFR_API int32_t sdfr_render_rays_per_lane(const SdfrGrid* grid, const SdfrCam* cam,
                                           int32_t n_envs);

/* Chooses the tile order of later renders on this handle (SDFR_ORDER_*,
 * default SDFR_ORDER_LOOKAHEAD). The lookahead order costs two small sort
 * launches per render, so it applies only to renders of at least
 * `min_tiles` tiles of 16x4 pixels (< 0: the library default, 65536 = 512 envs of
 * 128x64; 0: always); smaller renders take the launch order. Applies to the
 * tiles schedule and the surf-mask variant; results do not depend on it.
 * Synchronous; 0 or < 0. No reference counterpart. */
SDFR_API int32_t sdfr_grid_set_tile_order(SdfrGrid* grid, int32_t order, int64_t min_tiles);

/* Chooses when later renders on this handle read border voxels from the
 * face copies (SDFR_FACES_*, default SDFR_FACES_AUTO). A sample outside the
 * grid clamps to a border voxel (vision.py:104-106); on open scenes that is
 * 37-42% of all samples, and a face copy keeps a border layer's voxels 32
 * (fp32) or 64 (fp16) to a 128-byte line where the bricks hold 4-16. Only
 * the one-ray-per-lane march reads them; the copies hold the bricks'
 * values, so results do not depend on the mode. -3 for SDFR_FACES_ON on a
 * grid without copies (r16, or the linear layout). Synchronous; 0 or < 0.
 * No reference counterpart. */
SDFR_API int32_t sdfr_grid_set_border_faces(SdfrGrid* grid, int32_t mode);

/* Measurement hook, no reference counterpart: with a pair of the caller's
 * HIP events set (hipEvent_t, both or neither), every later render on this
 * handle records `start` on its stream right before the march kernel and
 * `stop` right after it, so hipEventElapsedTime(start, stop) is the march's
 * own duration (the ray-setup and tile-sort launches fall outside). The
 * events must stay valid while set; nulls clear them. Synchronous; 0 or < 0. */
SDFR_API int32_t sdfr_grid_set_march_events(SdfrGrid* grid, void* start, void* stop);

/* Bytes of device memory the handle's grid copy occupies (r16: codes and
 * brick headers; f32/f16 bricks: the bricks and the face copies). */
SDFR_API int64_t sdfr_grid_bytes(const SdfrGrid* grid);

/* Device bytes of the workspace sdfr_render needs for n_envs envs of this
 * camera: per env (W + H + 4) float2 of ray tables, then for the tile order
 * one int32, one uint16 and one uint32 per tile (16x4 pixels; tiles come in
 * 2x2 quads, ceil(W/32) * ceil(H/8) * 4 per env; each part 256-byte
 * aligned). < 0 on bad arguments. The tile order's bucket counts live in
 * the grid handle. */
SDFR_API int64_t sdfr_workspace_bytes(const SdfrCam* cam, int32_t n_envs);

/* Renders N depth images: equiangular (or pinhole) rays from each env's eye,
 * nearest-neighbour sphere trace through the grid, near-linear/far-compressed
 * encoding. Replaces GpuLidar._render_triton + _march_kernel
 * (vision.py:552-594, 59-116); results are per-ray and independent of N and
 * of how rays are scheduled. `workspace` is caller-owned device memory of at
 * least sdfr_workspace_bytes() bytes, 8-byte aligned; its contents need no
 * initialisation and are dead after the call. Asynchronous on `stream`;
 * allocates nothing. Returns 0, or < 0 with sdfr_last_error() set (bad
 * handle/argument, launch failure). */
SDFR_API int32_t sdfr_render(const SdfrGrid* grid, const SdfrCam* cam,
                             const SdfrPoses* poses, const SdfrImage* image,
                             void* workspace, int64_t workspace_size, void* stream);

/* Size of the device array sdfr_render_noalloc uses as its workspace: the
 * sdfr_workspace_bytes() of 8192 envs of 128x64 (23,330,816 bytes) fits. */
#define SDFR_NOALLOC_SCRATCH_BYTES (24ll << 20)

/* sdfr_render without a workspace argument and without any allocation: no
 * counterpart in the reference. For callers that cannot allocate device
 * memory — code under hipGraph capture, tight serving loops, harnesses that
 * forbid hipMalloc. The workspace is a static device array of
 * SDFR_NOALLOC_SCRATCH_BYTES that each GPU holds until the process ends;
 * renders whose sdfr_workspace_bytes() exceed it are refused (-2) before any
 * launch. Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other threads, other handles) race and must be
 * serialised by the caller. The grid's device must be current. The array's
 * address on a device is looked up by the first sdfr_grid_create there, so
 * a process's very first call may already be inside a graph capture.
 * Otherwise as sdfr_render: asynchronous on `stream`, 0 or < 0 with
 * sdfr_last_error(). */
SDFR_API int32_t sdfr_render_noalloc(const SdfrGrid* grid, const SdfrCam* cam,
                                     const SdfrPoses* poses, const SdfrImage* image,
                                     void* stream);

/* Reads the handle's grid copy back as nz*ny*nx fp32 values in [nz][ny][nx]
 * order: exactly the values the march samples (fp16 widened, r16 decoded).
 * The reference's kernel samples its device tensor GpuLidar.sdf_flat
 * (vision.py:476-480), which its tests read (tests/python/
 * test_lidar_march.py:130-138); this is the same view of this library's
 * private copy. `out`: device memory. Asynchronous on `stream`; 0 or < 0. */
SDFR_API int32_t sdfr_grid_read(const SdfrGrid* grid, float* out, void* stream);

/* Writes the unit direction of every ray, dirs[n][r][c][0..2] (dense f32),
 * with the same code the march uses to cast it; origin and ducked are not
 * read. The reference exposes the same quantity on its CPU path as
 * GpuLidar._dirs_equiangular / _dirs_pinhole (vision.py:596-624), which its
 * camera tests inspect (tests/python/test_pinhole.py:36-41). Asynchronous on
 * `stream`. */
SDFR_API int32_t sdfr_ray_dirs(const SdfrCam* cam, const SdfrPoses* poses, float* dirs,
                               void* stream);

/* ---- SDF bake ------------------------------------------------------------
 * Exact Euclidean distance transform of an occupancy grid: what the
 * reference's build_sdf computes with scipy (vision.py:428-438): pad one
 * layer of solid around the grid, distance_transform_edt(occ == 0,
 * sampling=cell), crop. `occ` is nz*ny*nx bytes in [nz][ny][nx] order on the
 * device (nonzero = solid); `out` receives nz*ny*nx distances in map units
 * (SDFR_F32 or SDFR_F16, rounded once from fp64), 0 in solid voxels.
 * Bit-identical to the reference's bake for power-of-two cells.
 * `workspace`: sdfr_edt_workspace_bytes() bytes of device memory, 8-byte
 * aligned. Asynchronous on `stream`; 0 or < 0 (sdfr_edt_last_error()). */
SDFR_API int64_t sdfr_edt_workspace_bytes(int32_t nx, int32_t ny, int32_t nz);
SDFR_API int32_t sdfr_edt(const uint8_t* occ, int32_t nx, int32_t ny, int32_t nz, float cell,
                          void* out, int32_t out_dtype, void* workspace, int64_t workspace_size,
                          void* stream);
SDFR_API const char* sdfr_edt_last_error(void);

/* ---- Goal field ----------------------------------------------------------
 * Geodesic distance to a goal zone over the free voxels of an occupancy grid:
 * the reference's build_goal_field bake (python/surfgym/goalfield.py:159-298)
 * and GoalField.sample (goalfield.py:68-94). The reference has no C ABI for
 * either (the bake is torch tensor ops, the sampler numpy); these are the
 * entry points its Python would bind.
 *
 * sdfr_goal_bake: `occ` is nz*ny*nx bytes [nz][ny][nx] on the device
 * (nonzero = solid). Distance 0 on the free voxels of the seed box
 * seed_lo..seed_hi (voxel indices x,y,z, inclusive, host arrays; clipped to
 * the grid — the reference's _zone_seed_box rounding, goalfield.py:148-156,
 * 228-231, is the caller's), relaxed over the 26 neighbours with edge cost
 * f32(cell * |offset|) in fp32 to the exact fixpoint, solid voxels excluded.
 * Then sentinel = reach_max + 2*cell replaces unreachable and solid voxels and
 * the field is quantised to uint16 at quant = cell/8 (goalfield.py:272-297).
 * Outputs (either may be NULL, not both): grid_q, the uint16 grid of the
 * reference's cache file; grid, its f32 dequantisation u16 * quant (what
 * GoalField holds). `workspace`: sdfr_goal_workspace_bytes() bytes of device
 * memory, 64-byte aligned. Synchronises `stream` (the host reads the
 * wavefront's queue length every few sweeps). Returns 0; -5 no free seed
 * voxel, -6 sentinel beyond the uint16 range, -7 not converged within
 * max_sweeps (sdfr_goal_last_error()). */
typedef struct SdfrGoalInfo {
    float reach_max;     /* largest finite geodesic distance, map units */
    float sentinel;      /* f32(reach_max + 2*cell) */
    float quant;         /* f32(cell / 8) */
    int32_t sweeps;      /* wavefront sweeps that visited at least one tile */
    int64_t n_seed;      /* free voxels in the seed box */
    int64_t tile_visits; /* 8x8x8 tile visits over all sweeps */
} SdfrGoalInfo;

SDFR_API int64_t sdfr_goal_workspace_bytes(int32_t nx, int32_t ny, int32_t nz);
SDFR_API int32_t sdfr_goal_bake(const uint8_t* occ, int32_t nx, int32_t ny, int32_t nz, float cell,
                                const int32_t* seed_lo, const int32_t* seed_hi, int32_t max_sweeps,
                                uint16_t* grid_q, float* grid, SdfrGoalInfo* info, void* workspace,
                                int64_t workspace_size, void* stream);

/* sdfr_goal_sample: trilinear distance at n positions over the honest corners
 * (value < f32(reach_max + cell/2)) of `grid` (SDFR_F32, or SDFR_U16 read as
 * u16 * quant), weights renormalised, f32(reach_max + 2*cell) where no corner
 * is honest — GoalField.sample bit for bit. `pos`: device rows of 3
 * (SDFR_F32 or SDFR_F64) at `pos_stride` elements; `mins` (host, 3 doubles)
 * and `cell` are the grid's placement. Asynchronous on `stream`. */
SDFR_API int32_t sdfr_goal_sample(const void* grid, int32_t grid_dtype, float quant, int32_t nx,
                                  int32_t ny, int32_t nz, const double* mins, double cell,
                                  double reach_max, const void* pos, int32_t pos_dtype,
                                  int64_t pos_stride, int64_t n, float* out, void* stream);
SDFR_API const char* sdfr_goal_last_error(void);

/* Message of the calling thread's most recent error ("" if none). */
SDFR_API const char* sdfr_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* SDFR_H */
