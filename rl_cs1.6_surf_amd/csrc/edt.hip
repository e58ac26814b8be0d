// edt.hip — exact Euclidean distance transform of a voxel occupancy grid on
// the GPU: the SDF bake of the reference's build_sdf (python/surfgym/vision.py
// :428-438), which pads the occupancy with one layer of solid and calls
//   scipy.ndimage.distance_transform_edt(occ == 0, sampling=cell)
// then crops the padding and stores f32 (f16 above 100 M voxels).
//
// Method: the squared distance transform is separable (Felzenszwalb &
// Huttenlocher, "Distance Transforms of Sampled Functions", 2012). Three
// passes:
//   x: one wave per row: each voxel's distance to the nearest solid in its
//      row (the padding makes x = -1 and x = nx solid), squared: g^2;
//   y: one thread per column: lower envelope of the parabolas
//      f(q) + (y - q)^2 over the column, with the padded rows q = -1 and
//      q = ny at f = 0;
//   z: the same along z, then d = sqrt(D * cell^2) in fp64, rounded once.
// All envelope arithmetic is exact integer arithmetic (squared distances in
// voxel units fit in int32, intersection comparisons are cross-multiplied in
// int64), so the squared distance of every voxel is exact. For a power-of-two
// cell (every cell pick_cell chooses, vision.py:283-298) scipy's float64
// sum of per-axis squares equals cell^2 * D exactly, so the result is
// bit-identical to the reference's bake.
//
// The y and z passes have two implementations with identical results: the
// envelope walk above (one thread per line) for passes with many lines, and
// a windowed exact search per output (edt_window) for passes with few.
//
// Scratch: two int32 planes of the grid and one uint64 envelope stack per
// line (~16 bytes per voxel, sdfr_edt_workspace_bytes).

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

#include "../../include/sdfr.h"

namespace {

thread_local char e_err[256];

__attribute__((format(printf, 2, 3))) int32_t efail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(e_err, sizeof e_err, fmt, ap);
    va_end(ap);
    return code;
}

// fp64 -> fp16, rounded once to nearest even (numpy's astype(float16)):
// round to fp32 toward zero and set the sticky bit if anything was dropped
// (round-to-odd keeps enough bits for the second rounding to be exact), then
// round that to fp16.
__device__ __forceinline__ __half f64_to_f16_rne(double x) {
    float t = __double2float_rz(x);
    if ((double)t != x) t = __uint_as_float(__float_as_uint(t) | 1u);
    return __float2half_rn(t);
}

// Pass x: per row, distance to the nearest solid (pads at -1 and nx), squared.
// One wave per row; lane l owns the run x in [l*C, (l+1)*C), C = ceil(nx/64).
// The nearest solid at or left of x is the last solid in the lane's run up to
// x, else the last solid of any lower lane (a prefix max over the wave), else
// the pad at -1; the right side mirrors it with a suffix min and the pad at nx.
__global__ __launch_bounds__(256) void edt_rows(const uint8_t* __restrict__ occ, int32_t* __restrict__ g,
                                                int nx, int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;   // uniform per wave
    const int lane = threadIdx.x & 63;
    const int C = (nx + 63) >> 6;
    const int x0 = min(lane * C, nx), x1 = min(x0 + C, nx);
    const uint8_t* o = occ + row * nx;
    int32_t* out = g + row * nx;
    int first = nx, last = -1;   // solids in this lane's run
    for (int x = x0; x < x1; ++x)
        if (o[x]) {
            first = min(first, x);
            last = x;
        }
    // inclusive scans over the wave: max of `last` up from lane 0, min of
    // `first` down from lane 63
    int lmax = last, rmin = first;
    for (int off = 1; off < 64; off <<= 1) {
        const int up = __shfl_up(lmax, off);
        const int dn = __shfl_down(rmin, off);
        if (lane >= off) lmax = max(lmax, up);
        if (lane + off < 64) rmin = min(rmin, dn);
    }
    int left = __shfl_up(lmax, 1);     // last solid below this lane's run
    int right = __shfl_down(rmin, 1);  // first solid above it
    if (lane == 0) left = -1;
    if (lane == 63) right = nx;
    for (int x = x0; x < x1; ++x) {
        if (o[x]) left = x;
        out[x] = x - left;
    }
    for (int x = x1 - 1; x >= x0; --x) {
        if (o[x]) right = x;
        const int32_t m = min(out[x], right - x);
        out[x] = m * m;
    }
}

// One column of the lower-envelope pass. The column has n real samples at
// stride `stride` from `f`, plus pad samples q = -1 and q = n with value 0.
// A parabola rooted at p is kept as (p, H) with H = f(p) + p^2, so the
// intersection of the parabolas rooted at a < b is
//   s(a, b) = (H_b - H_a) / (2 (b - a)),
// compared as cross-multiplied int64 fractions (exact). The envelope stack
// lives in `v` (stride `vstride`), one uint64 per vertex: H << 16 | (p + 1)
// (H < 2^32 and p + 1 < 2^16 under sdfr_edt's size checks); its top two
// vertices are kept in registers, so popping one costs a single dependent
// load, and the next sample is fetched while the current one is placed.
__device__ __forceinline__ int64_t fval(const int32_t* f, int64_t stride, int n, int q) {
    return (q < 0 || q >= n) ? 0 : (int64_t)f[(int64_t)q * stride];
}

struct Vtx {
    int p;       // root
    int64_t h;   // f(p) + p^2
};

__device__ __forceinline__ uint64_t pack_vtx(Vtx a) {
    return ((uint64_t)a.h << 16) | (uint64_t)(a.p + 1);
}

__device__ __forceinline__ Vtx unpack_vtx(uint64_t w) {
    return Vtx{(int)(w & 0xffffu) - 1, (int64_t)(w >> 16)};
}

__device__ __forceinline__ void envelope_line(const int32_t* __restrict__ f, int64_t stride, int n,
                                              uint64_t* __restrict__ v, int64_t vstride,
                                              int32_t* __restrict__ out, int64_t ostride,
                                              bool last, float* __restrict__ fout,
                                              __half* __restrict__ hout, double cell2) {
    // build the envelope over q = -1 .. n
    int k = 0;                          // index of the top vertex
    Vtx top{-1, 1};                     // the pad at q = -1: f = 0
    Vtx second{0, 0};                   // valid while k >= 1
    v[0] = pack_vtx(top);
    // the samples come in chunks of kChunk, the next chunk's loads in flight
    // while this one is placed (they do not depend on the envelope)
    constexpr int kChunk = 16;
    int64_t fc[kChunk], fn[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) fc[i] = fval(f, stride, n, i);
    for (int q0 = 0; q0 <= n; q0 += kChunk) {
#pragma unroll
        for (int i = 0; i < kChunk; ++i) fn[i] = fval(f, stride, n, q0 + kChunk + i);
#pragma unroll
        for (int i = 0; i < kChunk; ++i) {
            const int q = q0 + i;
            if (q > n) break;
            const int64_t hq = fc[i] + (int64_t)q * q;
            while (k > 0) {
                // pop the top while q's parabola takes over at or before the
                // point where the top took over from the vertex below it:
                // s(top, q) <= s(second, top)
                const int64_t s_num = hq - top.h, s_den = 2 * (int64_t)(q - top.p);
                const int64_t z_num = top.h - second.h, z_den = 2 * (int64_t)(top.p - second.p);
                if (s_num * z_den > z_num * s_den) break;
                --k;
                top = second;
                if (k > 0) second = unpack_vtx(v[(int64_t)(k - 1) * vstride]);
            }
            ++k;
            second = top;
            top = Vtx{q, hq};
            v[(int64_t)k * vstride] = pack_vtx(top);
        }
#pragma unroll
        for (int i = 0; i < kChunk; ++i) fc[i] = fn[i];
    }
    // read the envelope at the real samples; vertices j .. j+3 in registers
    // (w[0] current, w[1] next), the later ones loaded ahead of their use
    int j = 0;
    uint64_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = i <= k ? v[(int64_t)i * vstride] : 0;
    Vtx cur = unpack_vtx(w[0]);
    for (int q = 0; q < n; ++q) {
        while (j < k) {
            // advance while the next vertex takes over before q: s(cur, nxt) < q
            const Vtx nxt = unpack_vtx(w[1]);
            const int64_t z_num = nxt.h - cur.h, z_den = 2 * (int64_t)(nxt.p - cur.p);
            if (z_num >= (int64_t)q * z_den) break;
            ++j;
            cur = nxt;
            w[1] = w[2];
            w[2] = w[3];
            w[3] = j + 3 <= k ? v[(int64_t)(j + 3) * vstride] : 0;
        }
        const int64_t d = (int64_t)(q - cur.p) * (q - cur.p) + (cur.h - (int64_t)cur.p * cur.p);
        if (!last) {
            out[(int64_t)q * ostride] = (int32_t)d;
        } else {
            const double dist = sqrt((double)d * cell2);
            if (fout) fout[(int64_t)q * ostride] = (float)dist;
            else hout[(int64_t)q * ostride] = f64_to_f16_rne(dist);
        }
    }
}

// Pass y: one thread per (z, x) column of a [nz][ny][nx] plane array.
__global__ __launch_bounds__(256) void edt_cols(const int32_t* __restrict__ f, int32_t* __restrict__ out,
                                                uint64_t* __restrict__ v, int nx, int ny, int nz) {
    const int64_t line = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lines = (int64_t)nz * nx;
    if (line >= lines) return;
    const int z = (int)(line / nx), x = (int)(line - (int64_t)z * nx);
    const int64_t base = (int64_t)z * ny * nx + x;
    // envelope stack: entry j of this line at v[j*lines + line] (coalesced)
    envelope_line(f + base, nx, ny, v + line, lines, out + base, nx, false, nullptr, nullptr, 0.0);
}

// Pass z: one thread per (y, x) line; writes the distances.
__global__ __launch_bounds__(256) void edt_slabs(const int32_t* __restrict__ f, uint64_t* __restrict__ v,
                                                 float* __restrict__ fout, __half* __restrict__ hout,
                                                 int nx, int ny, int nz, double cell2) {
    const int64_t line = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lines = (int64_t)ny * nx;
    if (line >= lines) return;
    const int64_t plane = (int64_t)ny * nx;
    envelope_line(f + line, plane, nz, v + line, lines, nullptr, plane, true,
                  fout ? fout + line : nullptr, hout ? hout + line : nullptr, cell2);
}

// ---------------------------------------------------------- windowed passes --
// The y and z passes again, as a search per output instead of a walk per
// line: D(q) = min over p of f(p) + (q - p)^2, with the pads f(-1) = f(n) = 0.
// Starting from p = q (which gives f(q)), the candidates at distance d on
// either side are tried for d = 1, 2, ... while d^2 < best: a candidate at
// distance d adds at least d^2, so none further out can win, and the answer
// is exact. The pads bound best by min(q + 1, n - q)^2, so the search never
// leaves [-1, n]. A workgroup stages T whole lines (a tile of neighbouring
// columns) in LDS, entry (p + 1) * T + c for line c, and a wave works on
// 64 / T consecutive outputs of all T lines, whose searches are about equally
// long (neighbouring voxels have similar distances). The work is the sum of
// the distances in voxels; tens of thousands of waves are in flight instead
// of one per 64 lines.
//
// Lines of tile (bx, by): pass y (AXIS 1) lines (z = by, x), element p at
// (z*ny + p)*nx + x; pass z (AXIS 2) lines (y, x), y in [by*ty, by*ty + ty),
// element p at (p*ny + y)*nx + x. In both, x in [bx*tx, bx*tx + tx), T = tx*ty.
template <int AXIS, bool LAST>
__global__ __launch_bounds__(256) void edt_window(const int32_t* __restrict__ f,
                                                  int32_t* __restrict__ out,
                                                  float* __restrict__ fout,
                                                  __half* __restrict__ hout, int nx, int ny,
                                                  int nz, int tx, int ty, double cell2) {
    extern __shared__ int32_t s[];
    const int T = tx * ty;
    const int n = AXIS == 1 ? ny : nz;
    const int64_t stride = AXIS == 1 ? (int64_t)nx : (int64_t)nx * ny;
    const int x0 = blockIdx.x * tx;
    const int by = blockIdx.y;
    // element p of tile line c, or -1 for a line outside the grid
    auto line_base = [&](int c) -> int64_t {
        const int x = x0 + c % tx;
        if (x >= nx) return -1;
        if (AXIS == 1) return (int64_t)by * ny * nx + x;
        const int y = by * ty + c / tx;
        return y < ny ? (int64_t)y * nx + x : -1;
    };
    for (int i = threadIdx.x; i < (n + 2) * T; i += blockDim.x) {
        const int p = i / T - 1, c = i - (i / T) * T;
        const int64_t b = line_base(c);
        s[i] = (p < 0 || p >= n || b < 0) ? 0 : f[b + (int64_t)p * stride];
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n * T; i += blockDim.x) {
        const int q = i / T, c = i - (i / T) * T;
        const int32_t* col = s + c;
        int32_t best = col[(q + 1) * T];
        for (int d = 1; d * d < best; ++d) {
            const int32_t d2 = d * d;
            best = min(best, col[(q + 1 - d) * T] + d2);
            best = min(best, col[(q + 1 + d) * T] + d2);
        }
        const int64_t b = line_base(c);
        if (b < 0) continue;
        const int64_t o = b + (int64_t)q * stride;
        if constexpr (!LAST) {
            out[o] = best;
        } else {
            const double dist = sqrt((double)best * cell2);
            if (fout) fout[o] = (float)dist;
            else hout[o] = f64_to_f16_rne(dist);
        }
    }
}

// LDS budget of one windowed tile: a few workgroups per CU.
constexpr int64_t kWindowLds = 40 << 10;

// Which algorithm a pass takes. The envelope walk costs a fixed number of
// serial steps per line, so it is fast once there are lines enough to keep
// every SIMD busy; the windowed search costs the distances themselves but
// spreads them over many waves. Measured (one MI355X): on the 256x256x128
// ramp_field occupancy (32,768 y lines, 65,536 z lines) the windowed passes
// take 105 + 66 us against 514 + 243 us; on the 1024x1024x256 winding_track
// occupancy (262,144 y lines, 1,048,576 z lines; large open spaces) the
// envelope takes 5.7 + 2.8 ms against 9.4 + 3.8 ms. The windowed search
// runs while a pass has fewer lines than two waves per SIMD of envelope
// threads: 512 lines per CU.
constexpr int64_t kEnvelopeLinesPerCU = 512;

// Tile shape (tx, ty) of a windowed pass over `lines` lines of length n, or
// (0, 0) for the envelope kernels: when the lines are many enough, or when
// even four lines do not fit the LDS budget.
void window_tile(int n, int64_t lines, int cus, bool z_pass, int* tx, int* ty) {
    static const int shapes[][2] = {{16, 2}, {16, 1}, {8, 1}, {4, 1}};
    *tx = *ty = 0;
    if (cus > 0 && lines >= kEnvelopeLinesPerCU * cus) return;
    for (const auto& sh : shapes) {
        if (!z_pass && sh[1] != 1) continue;
        if ((int64_t)(n + 2) * sh[0] * sh[1] * (int64_t)sizeof(int32_t) <= kWindowLds) {
            *tx = sh[0];
            *ty = sh[1];
            return;
        }
    }
}

// Two int32 planes of the grid, then (8-byte aligned) the uint64 envelope
// stacks of the longer of the y and z passes.
int64_t edt_env_offset(int nx, int ny, int nz) {
    const int64_t vox = (int64_t)nx * ny * nz;
    return (2 * vox * (int64_t)sizeof(int32_t) + 7) & ~(int64_t)7;
}

int64_t edt_scratch_bytes(int nx, int ny, int nz) {
    const int64_t lines_y = (int64_t)nz * nx, lines_z = (int64_t)ny * nx;
    const int64_t venv = lines_y * (ny + 2) > lines_z * (nz + 2) ? lines_y * (ny + 2)
                                                                 : lines_z * (nz + 2);
    return edt_env_offset(nx, ny, nz) + venv * (int64_t)sizeof(uint64_t);
}

}  // namespace

extern "C" {

SDFR_API int64_t sdfr_edt_workspace_bytes(int32_t nx, int32_t ny, int32_t nz) {
    if (nx <= 0 || ny <= 0 || nz <= 0) return -2;
    return edt_scratch_bytes(nx, ny, nz);
}

SDFR_API const char* sdfr_edt_last_error(void) { return e_err; }

SDFR_API int32_t sdfr_edt(const uint8_t* occ, int32_t nx, int32_t ny, int32_t nz, float cell,
                          void* out, int32_t out_dtype, void* workspace, int64_t workspace_size,
                          void* stream) {
    e_err[0] = '\0';
    if (!occ || !out || !workspace) return efail(-1, "sdfr_edt: null pointer argument");
    if (nx <= 0 || ny <= 0 || nz <= 0)
        return efail(-2, "sdfr_edt: grid dims must be positive (got %d x %d x %d)", nx, ny, nz);
    if ((int64_t)nx + 2 > 46340 || (int64_t)ny + 2 > 46340 || (int64_t)nz + 2 > 46340)
        return efail(-2, "sdfr_edt: an axis longer than 46338 voxels overflows int32 distances");
    if ((int64_t)(nx + 2) * (nx + 2) + (int64_t)(ny + 2) * (ny + 2) + (int64_t)(nz + 2) * (nz + 2) >
        0x7fffffffLL)
        return efail(-2, "sdfr_edt: squared diagonal overflows int32");
    if (!(cell > 0.0f) || !isfinite(cell)) return efail(-2, "sdfr_edt: cell must be positive");
    if (out_dtype != SDFR_F32 && out_dtype != SDFR_F16)
        return efail(-3, "sdfr_edt: output dtype must be f32 or f16 (got %d)", out_dtype);
    const int64_t need = edt_scratch_bytes(nx, ny, nz);
    if (workspace_size < need)
        return efail(-2, "sdfr_edt: workspace of %lld bytes needed (got %lld)", (long long)need,
                     (long long)workspace_size);
    if (((uintptr_t)workspace & 7u) != 0) return efail(-2, "sdfr_edt: workspace must be 8-byte aligned");
    const int64_t vox = (int64_t)nx * ny * nz;
    int32_t* a = (int32_t*)workspace;
    int32_t* b = a + vox;
    uint64_t* v = (uint64_t*)((char*)workspace + edt_env_offset(nx, ny, nz));
    hipStream_t st = (hipStream_t)stream;
    const double cell2 = (double)cell * (double)cell;
    const int64_t rows = (int64_t)nz * ny, cols = (int64_t)nz * nx, lines = (int64_t)ny * nx;
    float* fout = out_dtype == SDFR_F32 ? (float*)out : nullptr;
    __half* hout = out_dtype == SDFR_F16 ? (__half*)out : nullptr;
    edt_rows<<<(int)((rows + 3) / 4), 256, 0, st>>>(occ, a, nx, rows);
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 0;   // unknown: the windowed passes wherever they fit
    int tx, ty;
    window_tile(ny, cols, cus, false, &tx, &ty);
    if (tx) {
        const dim3 grid((unsigned)((nx + tx - 1) / tx), (unsigned)nz);
        edt_window<1, false><<<grid, 256, (size_t)(ny + 2) * tx * ty * sizeof(int32_t), st>>>(
            a, b, nullptr, nullptr, nx, ny, nz, tx, ty, 0.0);
    } else {
        edt_cols<<<(int)((cols + 255) / 256), 256, 0, st>>>(a, b, v, nx, ny, nz);
    }
    window_tile(nz, lines, cus, true, &tx, &ty);
    if (tx) {
        const dim3 grid((unsigned)((nx + tx - 1) / tx), (unsigned)((ny + ty - 1) / ty));
        edt_window<2, true><<<grid, 256, (size_t)(nz + 2) * tx * ty * sizeof(int32_t), st>>>(
            b, nullptr, fout, hout, nx, ny, nz, tx, ty, cell2);
    } else {
        edt_slabs<<<(int)((lines + 255) / 256), 256, 0, st>>>(b, v, fout, hout, nx, ny, nz,
                                                              cell2);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return efail(-4, "sdfr_edt: launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
