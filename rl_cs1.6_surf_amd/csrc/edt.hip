// edt.hip — exact Euclidean distance transform of a voxel occupancy grid on
// the GPU: the SDF bake of the reference's build_sdf (python/surfgym/vision.py
// :428-438), which pads the occupancy with one layer of solid and calls
//   scipy.ndimage.distance_transform_edt(occ == 0, sampling=cell)
// then crops the padding and stores f32 (f16 above 100 M voxels).
//
// Method: the squared distance transform is separable (Felzenszwalb &
// Huttenlocher, "Distance Transforms of Sampled Functions", 2012). Three
// passes, one thread per grid line:
//   x: two sweeps give each voxel its distance to the nearest solid in its
//      row (the padding makes x = -1 and x = nx solid): g^2;
//   y: lower envelope of the parabolas f(q) + (y - q)^2 over the column,
//      with the padded rows q = -1 and q = ny at f = 0;
//   z: the same along z, then d = sqrt(D * cell^2) in fp64, rounded once.
// All envelope arithmetic is exact integer arithmetic (squared distances in
// voxel units fit in int32, intersection comparisons are cross-multiplied in
// int64), so the squared distance of every voxel is exact. For a power-of-two
// cell (every cell pick_cell chooses, vision.py:283-298) scipy's float64
// sum of per-axis squares equals cell^2 * D exactly, so the result is
// bit-identical to the reference's bake.
//
// Scratch: two int32 planes of the grid and one int32 envelope array per
// line (3 x 4 bytes per voxel, sdfr_edt_workspace_bytes).

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
__global__ __launch_bounds__(256) void edt_rows(const uint8_t* __restrict__ occ, int32_t* __restrict__ g,
                                                int nx, int64_t rows) {
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const uint8_t* o = occ + row * nx;
    int32_t* out = g + row * nx;
    int32_t d = 0;   // distance to the last solid seen, the pad at x = -1 to start
    for (int x = 0; x < nx; ++x) {
        d = o[x] ? 0 : d + 1;
        out[x] = d;
    }
    d = 0;           // the pad at x = nx
    for (int x = nx - 1; x >= 0; --x) {
        d = o[x] ? 0 : d + 1;
        const int32_t m = out[x] < d ? out[x] : d;
        out[x] = m * m;
    }
}

// One column of the lower-envelope pass. The column has n real samples at
// stride `stride` from `f`, plus pad samples q = -1 and q = n with value 0.
// Envelope vertices are stored as q + 1 in v (stride `vstride`).
__device__ __forceinline__ int64_t fval(const int32_t* f, int64_t stride, int n, int q) {
    return (q < 0 || q >= n) ? 0 : (int64_t)f[(int64_t)q * stride];
}

// Parabola p is left of q's takeover point? The intersection of parabolas
// rooted at a < b is s(a,b) = ((f_b + b^2) - (f_a + a^2)) / (2(b - a)).
struct Frac {
    int64_t num, den;   // den > 0
};

__device__ __forceinline__ Frac inter(const int32_t* f, int64_t stride, int n, int a, int b) {
    Frac s;
    s.num = (fval(f, stride, n, b) + (int64_t)b * b) - (fval(f, stride, n, a) + (int64_t)a * a);
    s.den = 2 * (int64_t)(b - a);
    return s;
}

__device__ __forceinline__ void envelope_line(const int32_t* __restrict__ f, int64_t stride, int n,
                                              int32_t* __restrict__ v, int64_t vstride,
                                              int32_t* __restrict__ out, int64_t ostride,
                                              bool last, float* __restrict__ fout,
                                              __half* __restrict__ hout, double cell2) {
    // build the envelope over q = -1 .. n
    int k = 0;
    v[0] = -1 + 1;
    for (int q = 0; q <= n; ++q) {
        while (true) {
            const int p = v[(int64_t)k * vstride] - 1;
            const Frac s = inter(f, stride, n, p, q);
            if (k == 0) break;
            const int pp = v[(int64_t)(k - 1) * vstride] - 1;
            const Frac zk = inter(f, stride, n, pp, p);
            // s <= z[k]  <=>  s.num * zk.den <= zk.num * s.den
            if (s.num * zk.den <= zk.num * s.den) --k;
            else break;
        }
        ++k;
        v[(int64_t)k * vstride] = q + 1;
    }
    // read the envelope at the real samples
    int j = 0;
    for (int q = 0; q < n; ++q) {
        while (j < k) {
            const int a = v[(int64_t)j * vstride] - 1, b = v[(int64_t)(j + 1) * vstride] - 1;
            const Frac z = inter(f, stride, n, a, b);
            if (z.num < (int64_t)q * z.den) ++j;   // z[j+1] < q
            else break;
        }
        const int p = v[(int64_t)j * vstride] - 1;
        const int64_t d = (int64_t)(q - p) * (q - p) + fval(f, stride, n, p);
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
                                                int32_t* __restrict__ v, int nx, int ny, int nz) {
    const int64_t line = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lines = (int64_t)nz * nx;
    if (line >= lines) return;
    const int z = (int)(line / nx), x = (int)(line - (int64_t)z * nx);
    const int64_t base = (int64_t)z * ny * nx + x;
    // envelope scratch: entry j of this line at v[j*lines + line] (coalesced)
    envelope_line(f + base, nx, ny, v + line, lines, out + base, nx, false, nullptr, nullptr, 0.0);
}

// Pass z: one thread per (y, x) line; writes the distances.
__global__ __launch_bounds__(256) void edt_slabs(const int32_t* __restrict__ f, int32_t* __restrict__ v,
                                                 float* __restrict__ fout, __half* __restrict__ hout,
                                                 int nx, int ny, int nz, double cell2) {
    const int64_t line = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t lines = (int64_t)ny * nx;
    if (line >= lines) return;
    const int64_t plane = (int64_t)ny * nx;
    envelope_line(f + line, plane, nz, v + line, lines, nullptr, plane, true,
                  fout ? fout + line : nullptr, hout ? hout + line : nullptr, cell2);
}

int64_t edt_scratch_bytes(int nx, int ny, int nz) {
    const int64_t vox = (int64_t)nx * ny * nz;
    const int64_t lines_y = (int64_t)nz * nx, lines_z = (int64_t)ny * nx;
    const int64_t venv = lines_y * (ny + 2) > lines_z * (nz + 2) ? lines_y * (ny + 2)
                                                                 : lines_z * (nz + 2);
    return (2 * vox + venv) * (int64_t)sizeof(int32_t);
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
    if (((uintptr_t)workspace & 3u) != 0) return efail(-2, "sdfr_edt: workspace must be 4-byte aligned");
    const int64_t vox = (int64_t)nx * ny * nz;
    int32_t* a = (int32_t*)workspace;
    int32_t* b = a + vox;
    int32_t* v = b + vox;
    hipStream_t st = (hipStream_t)stream;
    const double cell2 = (double)cell * (double)cell;
    const int64_t rows = (int64_t)nz * ny, cols = (int64_t)nz * nx, lines = (int64_t)ny * nx;
    edt_rows<<<(int)((rows + 255) / 256), 256, 0, st>>>(occ, a, nx, rows);
    edt_cols<<<(int)((cols + 255) / 256), 256, 0, st>>>(a, b, v, nx, ny, nz);
    edt_slabs<<<(int)((lines + 255) / 256), 256, 0, st>>>(
        b, v, out_dtype == SDFR_F32 ? (float*)out : nullptr,
        out_dtype == SDFR_F16 ? (__half*)out : nullptr, nx, ny, nz, cell2);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return efail(-4, "sdfr_edt: launch failed: %s", hipGetErrorString(e));
    return 0;
}

}  // extern "C"
