// goal.hip — the goal field: geodesic distance to a goal zone over the free
// voxels of an occupancy grid, and its trilinear sampler.
//
// Reference: python/surfgym/goalfield.py. build_goal_field (:159-298) seeds
// d = 0 on the free voxels of the inflated goal box, then relaxes
//   d[v] = min(d[v], d[v + o] + w_o)   for the 26 neighbour offsets o,
//   w_o = f32(cell * sqrt(|o|^2)), solid voxels pinned at +inf,
// in fp32 until nothing changes (:228-270), takes reach_max = the largest
// finite distance, replaces +inf by sentinel = reach_max + 2*cell, and stores
// round(d / (cell/8)) as uint16 (:272-297). GoalField.sample (:68-94)
// trilinearly interpolates the dequantised grid over its "honest" corners
// (value < reach_max + cell/2) only.
//
// Exactness. x -> fl(x + w) is monotone, so every relaxation order that runs
// until nothing changes ends at the same values: for each voxel, the least
// fp32 left-to-right sum of edge weights over the paths from a seed. The bake
// therefore relaxes in the order that suits the GPU instead of the
// reference's whole-grid Jacobi sweeps (one voxel of progress per sweep):
//
//   * 8x8x8 tiles, one 512-thread block per tile visit, are loaded with a
//     one-voxel halo into LDS and relaxed there (Gauss-Seidel, in place)
//     until the tile is stable — a visit carries a front across a tile;
//   * a tile writes back only the voxels it lowered, in place, and queues
//     the neighbour tiles whose halo holds one of them (a tile is stable
//     against its halo after a visit, so nothing else needs revisiting);
//   * sweeps consume one queue and fill the next, without the host; the
//     host reads the next queue's length every few sweeps and stops when it
//     is empty. Concurrent visits may read a halo value before or after a
//     neighbour lowers it: both are path sums, and any lowering after a read
//     queues the reader again, so an empty queue means every voxel is stable
//     against all 26 neighbours — the fixpoint.
//
// Work is proportional to the tiles the front crosses (times how often
// corrections re-cross them), not to grid size times path length.

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/sdfr.h"

namespace {

thread_local char g_goal_err[256];

__attribute__((format(printf, 2, 3))) int32_t gfail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_goal_err, sizeof g_goal_err, fmt, ap);
    va_end(ap);
    return code;
}

constexpr int kT = 8;                    // tile edge (voxels)
constexpr int kH = kT + 2;               // tile edge with halo
constexpr int kHalo = kH * kH * kH;      // 1000 LDS floats
constexpr int kThreads = kT * kT * kT;   // one thread per tile voxel
constexpr int kMaxLocal = 96;            // local sweeps per visit; the tile is requeued if hit
constexpr int kSweepChunk = 32;          // sweeps launched between host checks

// control words after the queues (uint32)
enum { kCount0 = 0, kCount1 = 1, kCount2 = 2, kSeeds = 3, kReach = 4, kLastBusy = 5, kVisitsLo = 6,
       kVisitsHi = 7, kCtl = 8 };

struct GoalArgs {
    const uint8_t* occ;
    float* d;
    uint32_t* mark;       // [tiles] last sweep the tile was queued for
    uint32_t* queues;     // [3][tiles]
    uint32_t* ctl;        // [kCtl]
    int nx, ny, nz;
    int tx, ty, tz;       // tiles per axis
    uint32_t tiles;
    float w1, w2, w3;     // edge weights for |o|^2 = 1, 2, 3
};

// d = +inf everywhere, 0 on the free voxels of the seed box; the tiles that
// hold a seed or touch one through their halo form the first queue.
__global__ __launch_bounds__(256) void goal_init(GoalArgs a, int lx, int ly, int lz, int hx, int hy,
                                                 int hz, int tlx, int tly, int tlz, int thx, int thy,
                                                 int thz) {
    const int64_t vox = (int64_t)a.nx * a.ny * a.nz;
    uint32_t seeds = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vox;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int x = (int)(i % a.nx);
        const int64_t r = i / a.nx;
        const int y = (int)(r % a.ny), z = (int)(r / a.ny);
        const bool seed = x >= lx && x <= hx && y >= ly && y <= hy && z >= lz && z <= hz && !a.occ[i];
        a.d[i] = seed ? 0.0f : INFINITY;
        seeds += seed;
    }
    const int bnx = thx - tlx + 1, bny = thy - tly + 1;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < a.tiles;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int tx = (int)(t % a.tx);
        const int64_t r = t / a.tx;
        const int ty = (int)(r % a.ty), tz = (int)(r / a.ty);
        const bool in = tx >= tlx && tx <= thx && ty >= tly && ty <= thy && tz >= tlz && tz <= thz;
        a.mark[t] = in ? 1u : 0u;
        if (in) a.queues[1 * a.tiles + ((tz - tlz) * bny + (ty - tly)) * bnx + (tx - tlx)] = (uint32_t)t;
    }
    for (int off = 32; off > 0; off >>= 1) seeds += __shfl_down(seeds, off);
    if ((threadIdx.x & 63) == 0 && seeds) atomicAdd(&a.ctl[kSeeds], seeds);
}

__device__ __forceinline__ float relax_voxel(const float* s, int c, float m, float w1, float w2,
                                             float w3) {
#pragma unroll
    for (int oz = -1; oz <= 1; ++oz)
#pragma unroll
        for (int oy = -1; oy <= 1; ++oy)
#pragma unroll
            for (int ox = -1; ox <= 1; ++ox) {
                const int q = oz * oz + oy * oy + ox * ox;
                if (q == 0) continue;
                const float w = q == 1 ? w1 : (q == 2 ? w2 : w3);
                m = fminf(m, s[c + (oz * kH + oy) * kH + ox] + w);
            }
    return m;
}

// Sweep k: visit every tile of queue k%3, fill queue (k+1)%3, clear the
// count of queue (k+2)%3 (consumed by sweep k-1, filled by sweep k+1).
__global__ __launch_bounds__(kThreads) void goal_sweep(GoalArgs a, uint32_t k) {
    __shared__ float s[kHalo];
    __shared__ uint32_t s_push;
    const uint32_t qin = k % 3u, qout = (k + 1u) % 3u;
    const uint32_t n = a.ctl[qin];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        a.ctl[(k + 2u) % 3u] = 0u;
        if (n) {
            a.ctl[kLastBusy] = k;
            atomicAdd((unsigned long long*)&a.ctl[kVisitsLo], (unsigned long long)n);
        }
    }
    const uint32_t* qi = a.queues + (size_t)qin * a.tiles;
    uint32_t* qo = a.queues + (size_t)qout * a.tiles;
    const int tid = threadIdx.x;
    const int lx = tid & 7, ly = (tid >> 3) & 7, lz = tid >> 6;
    const int c = ((lz + 1) * kH + (ly + 1)) * kH + (lx + 1);
    for (uint32_t e = blockIdx.x; e < n; e += gridDim.x) {
        const uint32_t tile = qi[e];
        const int tx = (int)(tile % (uint32_t)a.tx);
        const uint32_t r = tile / (uint32_t)a.tx;
        const int ty = (int)(r % (uint32_t)a.ty), tz = (int)(r / (uint32_t)a.ty);
        const int x0 = tx * kT - 1, y0 = ty * kT - 1, z0 = tz * kT - 1;
        for (int i = tid; i < kHalo; i += kThreads) {
            const int hx = i % kH, hy = (i / kH) % kH, hz = i / (kH * kH);
            const int x = x0 + hx, y = y0 + hy, z = z0 + hz;
            float v = INFINITY;   // outside the grid: never lowers a neighbour
            if (x >= 0 && y >= 0 && z >= 0 && x < a.nx && y < a.ny && z < a.nz)
                v = a.d[((int64_t)z * a.ny + y) * a.nx + x];
            s[i] = v;
        }
        const int x = x0 + 1 + lx, y = y0 + 1 + ly, z = z0 + 1 + lz;
        const bool inside = x < a.nx && y < a.ny && z < a.nz;
        const int64_t idx = ((int64_t)z * a.ny + y) * a.nx + x;
        const bool open = inside && a.occ[idx] == 0;
        if (tid == 0) s_push = 0u;
        __syncthreads();
        const float start = s[c];
        // Gauss-Seidel in LDS: only this thread writes s[c]; a neighbour read
        // sees the old or the new value, both path sums. A local sweep in
        // which no voxel lowered saw a constant tile: the tile is stable.
        int moving = 1;
        int it = 0;
        while (moving && it < kMaxLocal) {
            int lowered = 0;
            if (open) {
                const float cur = s[c];
                const float m = relax_voxel(s, c, cur, a.w1, a.w2, a.w3);
                if (m < cur) {
                    s[c] = m;
                    lowered = 1;
                }
            }
            moving = __syncthreads_or(lowered);
            ++it;
        }
        const float fin = s[c];
        uint32_t bits = 0;
        if (fin < start) {
            a.d[idx] = fin;
            // neighbour tiles whose halo holds this voxel: per axis, offset 0
            // always, -1 on the tile's low face, +1 on its high face
            const int xs0 = lx == 0 ? -1 : 0, xs1 = lx == kT - 1 ? 1 : 0;
            const int ys0 = ly == 0 ? -1 : 0, ys1 = ly == kT - 1 ? 1 : 0;
            const int zs0 = lz == 0 ? -1 : 0, zs1 = lz == kT - 1 ? 1 : 0;
            for (int dz = zs0; dz <= zs1; ++dz)
                for (int dy = ys0; dy <= ys1; ++dy)
                    for (int dx = xs0; dx <= xs1; ++dx)
                        bits |= 1u << ((dz + 1) * 9 + (dy + 1) * 3 + (dx + 1));
            bits &= ~(1u << 13);
        }
        if (moving && tid == 0) bits |= 1u << 13;   // local cap hit: visit again
        if (bits) atomicOr(&s_push, bits);
        __syncthreads();
        const uint32_t push = s_push;
        if (tid < 27 && ((push >> tid) & 1u)) {
            const int dz = tid / 9 - 1, dy = (tid / 3) % 3 - 1, dx = tid % 3 - 1;
            const int ux = tx + dx, uy = ty + dy, uz = tz + dz;
            if (ux >= 0 && uy >= 0 && uz >= 0 && ux < a.tx && uy < a.ty && uz < a.tz) {
                const uint32_t u = ((uint32_t)uz * (uint32_t)a.ty + (uint32_t)uy) * (uint32_t)a.tx + (uint32_t)ux;
                if (atomicMax(&a.mark[u], k + 1u) < k + 1u) {
                    const uint32_t slot = atomicAdd(&a.ctl[qout], 1u);
                    qo[slot] = u;
                }
            }
        }
        __syncthreads();   // s and s_push are reused by the next visit
    }
}

// reach_max: the largest finite distance (non-negative floats order as their
// bit patterns). Four distances per load (the distances start the workspace,
// which the bake requires 64-byte aligned), the last vox % 4 one at a time;
// one atomic per block (atomics from every wave to the one word serialise).
constexpr int kReachBlocks = 512;
__global__ __launch_bounds__(256) void goal_reach_max(const float* d, int64_t vox, uint32_t* best) {
    __shared__ uint32_t s_m[4];
    uint32_t m = 0;
    const int64_t n4 = vox >> 2;
    const float4* d4 = reinterpret_cast<const float4*>(d);
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += step) {
        const float4 v = d4[i];
        if (v.x != INFINITY) m = max(m, __float_as_uint(v.x));
        if (v.y != INFINITY) m = max(m, __float_as_uint(v.y));
        if (v.z != INFINITY) m = max(m, __float_as_uint(v.z));
        if (v.w != INFINITY) m = max(m, __float_as_uint(v.w));
    }
    for (int64_t i = (n4 << 2) + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vox; i += step) {
        const float v = d[i];
        if (v != INFINITY) m = max(m, __float_as_uint(v));
    }
    for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_down(m, off));
    if ((threadIdx.x & 63) == 0) s_m[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = max(max(s_m[0], s_m[1]), max(s_m[2], s_m[3]));
        if (m) atomicMax(best, m);
    }
}

// +inf -> sentinel, then round(d / quant) clamped to [0, 65535]. The
// reference divides a CUDA tensor by a Python scalar, which torch evaluates as
// d * (1/quant) with the reciprocal rounded to fp32 (identical to d / quant
// for the power-of-two cells the reference picks), and rounds half to even.
__global__ __launch_bounds__(256) void goal_quantise(const float* d, int64_t vox, float sentinel,
                                                     float inv_quant, float quant, uint16_t* q_out,
                                                     float* g_out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < vox;
         i += (int64_t)gridDim.x * blockDim.x) {
        float v = d[i];
        if (v == INFINITY) v = sentinel;
        const float q = fminf(fmaxf(rintf(v * inv_quant), 0.0f), 65535.0f);
        const uint16_t u = (uint16_t)q;
        if (q_out) q_out[i] = u;
        if (g_out) g_out[i] = (float)u * quant;
    }
}

// GoalField.sample (goalfield.py:68-94): trilinear over the honest corners.
template <int GRID, int POS>
__global__ __launch_bounds__(256) void goal_sample(const void* __restrict__ grid, float quant, int nx,
                                                   int ny, int nz, double mnx, double mny, double mnz,
                                                   double cell, float valid_max, float sentinel,
                                                   const void* __restrict__ pos, int64_t pos_stride,
                                                   int64_t n, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    double p[3];
    for (int j = 0; j < 3; ++j)
        p[j] = POS == SDFR_F64 ? ((const double*)pos)[i * pos_stride + j]
                               : (double)((const float*)pos)[i * pos_stride + j];
    const double gx = (p[0] - mnx) / cell - 0.5;
    const double gy = (p[1] - mny) / cell - 0.5;
    const double gz = (p[2] - mnz) / cell - 0.5;
    const double fx0 = floor(gx), fy0 = floor(gy), fz0 = floor(gz);
    const float fx = (float)(gx - fx0), fy = (float)(gy - fy0), fz = (float)(gz - fz0);
    // corner indices clamped in double: a far-off position cannot overflow
    const double cx[2] = {fmin(fmax(fx0, 0.0), nx - 1.0), fmin(fmax(fx0 + 1.0, 0.0), nx - 1.0)};
    const double cy[2] = {fmin(fmax(fy0, 0.0), ny - 1.0), fmin(fmax(fy0 + 1.0, 0.0), ny - 1.0)};
    const double cz[2] = {fmin(fmax(fz0, 0.0), nz - 1.0), fmin(fmax(fz0 + 1.0, 0.0), nz - 1.0)};
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int dz = 0; dz < 2; ++dz)
#pragma unroll
        for (int dy = 0; dy < 2; ++dy)
#pragma unroll
            for (int dx = 0; dx < 2; ++dx) {
                const int64_t k = ((int64_t)cz[dz] * ny + (int64_t)cy[dy]) * nx + (int64_t)cx[dx];
                const float v = GRID == SDFR_F32 ? ((const float*)grid)[k]
                                                 : (float)((const uint16_t*)grid)[k] * quant;
                const float wx = dx ? fx : 1.0f - fx;
                const float wy = dy ? fy : 1.0f - fy;
                const float wz = dz ? fz : 1.0f - fz;
                const float w = ((wx * wy) * wz) * (v < valid_max ? 1.0f : 0.0f);
                num = num + w * v;
                den = den + w;
            }
    out[i] = den > 1e-6f ? num / fmaxf(den, 1e-6f) : sentinel;
}

struct Layout {
    int64_t vox, d_off, mark_off, q_off, ctl_off, total;
    uint32_t tiles;
};

Layout layout_of(int nx, int ny, int nz) {
    Layout l;
    l.vox = (int64_t)nx * ny * nz;
    const int64_t tiles = (int64_t)((nx + kT - 1) / kT) * ((ny + kT - 1) / kT) * ((nz + kT - 1) / kT);
    l.tiles = (uint32_t)tiles;
    l.d_off = 0;
    l.mark_off = l.d_off + l.vox * 4;
    l.q_off = l.mark_off + tiles * 4;
    l.ctl_off = l.q_off + 3 * tiles * 4;
    l.ctl_off = (l.ctl_off + 63) & ~(int64_t)63;
    l.total = l.ctl_off + kCtl * 4;
    return l;
}

}  // namespace

extern "C" {

SDFR_API const char* sdfr_goal_last_error(void) { return g_goal_err; }

SDFR_API int64_t sdfr_goal_workspace_bytes(int32_t nx, int32_t ny, int32_t nz) {
    if (nx <= 0 || ny <= 0 || nz <= 0) return -2;
    return layout_of(nx, ny, nz).total;
}

SDFR_API int32_t sdfr_goal_bake(const uint8_t* occ, int32_t nx, int32_t ny, int32_t nz, float cell,
                                const int32_t* seed_lo, const int32_t* seed_hi, int32_t max_sweeps,
                                uint16_t* grid_q, float* grid, SdfrGoalInfo* info, void* workspace,
                                int64_t workspace_size, void* stream) {
    g_goal_err[0] = '\0';
    if (!occ || !seed_lo || !seed_hi || !workspace || !info || (!grid_q && !grid))
        return gfail(-1, "sdfr_goal_bake: null pointer argument");
    if (nx <= 0 || ny <= 0 || nz <= 0)
        return gfail(-2, "sdfr_goal_bake: grid dims must be positive (got %d x %d x %d)", nx, ny, nz);
    if (!(cell > 0.0f) || !isfinite(cell)) return gfail(-2, "sdfr_goal_bake: cell must be positive");
    if (max_sweeps <= 0) return gfail(-2, "sdfr_goal_bake: max_sweeps must be positive");
    const int64_t tiles64 = (int64_t)((nx + kT - 1) / kT) * ((ny + kT - 1) / kT) * ((nz + kT - 1) / kT);
    if (tiles64 > 0x3fffffffLL) return gfail(-2, "sdfr_goal_bake: grid too large");
    const Layout L = layout_of(nx, ny, nz);
    if (workspace_size < L.total)
        return gfail(-2, "sdfr_goal_bake: workspace of %lld bytes needed (got %lld)",
                     (long long)L.total, (long long)workspace_size);
    if (((uintptr_t)workspace & 63u) != 0)
        return gfail(-2, "sdfr_goal_bake: workspace must be 64-byte aligned");
    // the seed box, clipped to the grid (goalfield.py:228-240)
    const int dims[3] = {nx, ny, nz};
    int lo[3], hi[3], tlo[3], thi[3];
    for (int j = 0; j < 3; ++j) {
        lo[j] = seed_lo[j] < 0 ? 0 : seed_lo[j];
        hi[j] = seed_hi[j] > dims[j] - 1 ? dims[j] - 1 : seed_hi[j];
        if (hi[j] < lo[j])
            return gfail(-5, "sdfr_goal_bake: goal zone contains no free voxel (empty seed box)");
        const int ntj = (dims[j] + kT - 1) / kT;
        tlo[j] = lo[j] == 0 ? 0 : (lo[j] - 1) / kT;
        thi[j] = (hi[j] + 1) / kT > ntj - 1 ? ntj - 1 : (hi[j] + 1) / kT;
    }
    hipStream_t st = (hipStream_t)stream;
    uint8_t* ws = (uint8_t*)workspace;
    GoalArgs g;
    g.occ = occ;
    g.d = (float*)(ws + L.d_off);
    g.mark = (uint32_t*)(ws + L.mark_off);
    g.queues = (uint32_t*)(ws + L.q_off);
    g.ctl = (uint32_t*)(ws + L.ctl_off);
    g.nx = nx;
    g.ny = ny;
    g.nz = nz;
    g.tx = (nx + kT - 1) / kT;
    g.ty = (ny + kT - 1) / kT;
    g.tz = (nz + kT - 1) / kT;
    g.tiles = L.tiles;
    // cell * sqrt(|o|^2) in float64 (Python floats), added to an fp32 tensor
    // as an fp32 scalar
    g.w1 = (float)((double)cell * sqrt(1.0));
    g.w2 = (float)((double)cell * sqrt(2.0));
    g.w3 = (float)((double)cell * sqrt(3.0));
    const uint32_t first = (uint32_t)(thi[0] - tlo[0] + 1) * (uint32_t)(thi[1] - tlo[1] + 1) *
                           (uint32_t)(thi[2] - tlo[2] + 1);
    uint32_t ctl0[kCtl] = {0, first, 0, 0, 0, 0, 0, 0};
    hipError_t e = hipMemcpyAsync(g.ctl, ctl0, sizeof ctl0, hipMemcpyHostToDevice, st);
    if (e != hipSuccess) return gfail(-4, "sdfr_goal_bake: %s", hipGetErrorString(e));
    int init_blocks = (int)((L.vox + 255) / 256);
    if (init_blocks > 8192) init_blocks = 8192;
    goal_init<<<init_blocks, 256, 0, st>>>(g, lo[0], lo[1], lo[2], hi[0], hi[1], hi[2], tlo[0], tlo[1],
                                           tlo[2], thi[0], thi[1], thi[2]);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 256;
    const int sweep_blocks = cus * 4;   // 4 x 512 threads fill a CU's wave slots
    uint32_t host[kCtl];
    uint32_t k = 1;
    bool done = false;
    while (!done && (int64_t)k <= max_sweeps) {
        for (int j = 0; j < kSweepChunk && (int64_t)k <= max_sweeps; ++j, ++k)
            goal_sweep<<<sweep_blocks, kThreads, 0, st>>>(g, k);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(host, g.ctl, sizeof host, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        if (e != hipSuccess) return gfail(-4, "sdfr_goal_bake: %s", hipGetErrorString(e));
        if (host[kSeeds] == 0)
            return gfail(-5, "sdfr_goal_bake: goal zone contains no free voxel");
        if (host[k % 3u] == 0) done = true;   // k is the next sweep: its queue is empty
    }
    if (!done) return gfail(-7, "sdfr_goal_bake: not converged after %d sweeps", max_sweeps);
    goal_reach_max<<<kReachBlocks, 256, 0, st>>>(g.d, L.vox, g.ctl + kReach);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipMemcpyAsync(host, g.ctl, sizeof host, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return gfail(-4, "sdfr_goal_bake: %s", hipGetErrorString(e));
    float reach_max;
    memcpy(&reach_max, &host[kReach], 4);
    // Python floats: sentinel = reach_max + 2*cell, quant = cell/8; stored fp32
    const double sentinel = (double)reach_max + 2.0 * (double)cell;
    const double quant = (double)cell / 8.0;
    info->reach_max = reach_max;
    info->sentinel = (float)sentinel;
    info->quant = (float)quant;
    info->sweeps = (int32_t)host[kLastBusy];
    info->n_seed = (int64_t)host[kSeeds];
    info->tile_visits = (int64_t)host[kVisitsLo] | ((int64_t)host[kVisitsHi] << 32);
    if (sentinel / quant > 65535.0)
        return gfail(-6, "sdfr_goal_bake: sentinel %.0fu exceeds the uint16 range at quant %gu",
                     sentinel, quant);
    const float quant_f = (float)quant;
    const float inv_quant = 1.0f / quant_f;
    goal_quantise<<<init_blocks, 256, 0, st>>>(g.d, L.vox, (float)sentinel, inv_quant, quant_f, grid_q,
                                               grid);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return gfail(-4, "sdfr_goal_bake: %s", hipGetErrorString(e));
    return 0;
}

SDFR_API int32_t sdfr_goal_sample(const void* grid, int32_t grid_dtype, float quant, int32_t nx,
                                  int32_t ny, int32_t nz, const double* mins, double cell,
                                  double reach_max, const void* pos, int32_t pos_dtype,
                                  int64_t pos_stride, int64_t n, float* out, void* stream) {
    g_goal_err[0] = '\0';
    if (!grid || !mins || !out || (!pos && n > 0))
        return gfail(-1, "sdfr_goal_sample: null pointer argument");
    if (nx <= 0 || ny <= 0 || nz <= 0 || n < 0 || !(cell > 0.0))
        return gfail(-2, "sdfr_goal_sample: bad dims, count or cell");
    if (grid_dtype != SDFR_F32 && grid_dtype != SDFR_U16)
        return gfail(-3, "sdfr_goal_sample: grid dtype must be f32 or u16 (got %d)", grid_dtype);
    if (pos_dtype != SDFR_F32 && pos_dtype != SDFR_F64)
        return gfail(-3, "sdfr_goal_sample: position dtype must be f32 or f64 (got %d)", pos_dtype);
    if (pos_stride < 3) return gfail(-2, "sdfr_goal_sample: position row stride below 3");
    if (n == 0) return 0;
    if (n > (int64_t)0x7fffffff * 256) return gfail(-2, "sdfr_goal_sample: too many positions");
    // GoalField.__init__ (goalfield.py:59-66): Python floats, compared in fp32
    const float sentinel = (float)(reach_max + 2.0 * cell);
    const float valid_max = (float)(reach_max + 0.5 * cell);
    const int blocks = (int)((n + 255) / 256);
    hipStream_t st = (hipStream_t)stream;
#define GOAL_SAMPLE(G, P)                                                                              \
    goal_sample<G, P><<<blocks, 256, 0, st>>>(grid, quant, nx, ny, nz, mins[0], mins[1], mins[2], cell, \
                                              valid_max, sentinel, pos, pos_stride, n, out)
    if (grid_dtype == SDFR_F32 && pos_dtype == SDFR_F64) GOAL_SAMPLE(SDFR_F32, SDFR_F64);
    else if (grid_dtype == SDFR_F32) GOAL_SAMPLE(SDFR_F32, SDFR_F32);
    else if (pos_dtype == SDFR_F64) GOAL_SAMPLE(SDFR_U16, SDFR_F64);
    else GOAL_SAMPLE(SDFR_U16, SDFR_F32);
#undef GOAL_SAMPLE
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return gfail(-4, "sdfr_goal_sample: launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
