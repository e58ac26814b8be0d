/* render_check.c — the renderer driven from plain C through include/sdfr.h,
 * with no Python and no torch: the way a C or C++ caller (or any FFI) binds
 * libsdfr.so. Test infrastructure: built and run by tests/test_gpu_c_abi.py.
 *
 * It builds an analytic distance grid on the host (distance in map units to
 * a floor and to two boxes, voxel-centre sampled), creates a grid handle
 * from host memory, renders N envs into device memory with a caller
 * workspace and with sdfr_render_noalloc, and compares both images value for
 * value with the CPU oracle (oracle/march.c, linked from
 * oracle/liboracle_march.so) on the same inputs. Prints one line and exits
 * 0 when everything matches.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "sdfr.h"

/* the oracle's entry point (oracle/march.c) */
int oracle_render(const float* grid, int nx, int ny, int nz, const float* mins, float cell, int W,
                  int H, int camera, double hfov, double vfov, double tan_h, double tan_v,
                  float range, float near, float hit_eps, float min_step, int max_steps,
                  const float* origin, const float* yaw, const float* pitch, const float* ducked,
                  int N, float* out, int32_t* loads, const int8_t* nzg, int nthreads);

#define CHECK(x)                                                                  \
    do {                                                                          \
        hipError_t e_ = (x);                                                      \
        if (e_ != hipSuccess) {                                                   \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,             \
                    hipGetErrorString(e_));                                       \
            return 2;                                                             \
        }                                                                         \
    } while (0)

static float box_dist(float x, float y, float z, const float lo[3], const float hi[3]) {
    const float dx = fmaxf(fmaxf(lo[0] - x, x - hi[0]), 0.0f);
    const float dy = fmaxf(fmaxf(lo[1] - y, y - hi[1]), 0.0f);
    const float dz = fmaxf(fmaxf(lo[2] - z, z - hi[2]), 0.0f);
    return sqrtf(dx * dx + dy * dy + dz * dz);
}

int main(void) {
    if (sdfr_abi_version() != SDFR_ABI_VERSION) {
        fprintf(stderr, "ABI %d, header %d\n", sdfr_abi_version(), SDFR_ABI_VERSION);
        return 2;
    }
    const int nx = 48, ny = 40, nz = 24, N = 6, W = 64, H = 32;
    const float cell = 16.0f, mins[3] = {-32.0f, -16.0f, -8.0f};
    const float b0lo[3] = {200.0f, 100.0f, 0.0f}, b0hi[3] = {300.0f, 260.0f, 120.0f};
    const float b1lo[3] = {420.0f, 300.0f, 40.0f}, b1hi[3] = {520.0f, 420.0f, 90.0f};
    const size_t nvox = (size_t)nx * ny * nz;
    float* grid = (float*)malloc(nvox * sizeof(float));
    for (int z = 0; z < nz; ++z)
        for (int y = 0; y < ny; ++y)
            for (int x = 0; x < nx; ++x) {
                const float px = mins[0] + (x + 0.5f) * cell, py = mins[1] + (y + 0.5f) * cell;
                const float pz = mins[2] + (z + 0.5f) * cell;
                float d = fmaxf(pz, 0.0f);                      /* the floor z <= 0 */
                d = fminf(d, box_dist(px, py, pz, b0lo, b0hi));
                d = fminf(d, box_dist(px, py, pz, b1lo, b1hi));
                grid[((size_t)z * ny + y) * nx + x] = d;
            }
    float origin[3 * 6], yaw[6], pitch[6], ducked[6];
    for (int n = 0; n < N; ++n) {
        origin[3 * n + 0] = 60.0f + 90.0f * n;
        origin[3 * n + 1] = 40.0f + 50.0f * n;
        origin[3 * n + 2] = 150.0f + 10.0f * n;
        yaw[n] = -150.0f + 61.0f * n;
        pitch[n] = -60.0f + 17.0f * n;
        ducked[n] = (float)(n & 1);
    }

    SdfrGridDesc desc = {nx, ny, nz, {mins[0], mins[1], mins[2]}, cell};
    char err[256];
    SdfrGrid* g = sdfr_grid_create(&desc, grid, SDFR_F32, 0 /* host */, SDFR_F32,
                                   SDFR_LAYOUT_BRICK4, NULL, err, sizeof err);
    if (!g) {
        fprintf(stderr, "sdfr_grid_create: %s\n", err);
        return 2;
    }
    const double tan_h = tan(60.0 * 3.14159265358979323846 / 180.0);
    const double tan_v = tan(45.0 * 3.14159265358979323846 / 180.0);
    SdfrCam cam = {W, H, 120.0, 90.0, tan_h, tan_v, 1200.0f, 700.0f, 9.6f, 4.8f, 64,
                   SDFR_CAM_EQUIANGULAR};

    float *d_origin, *d_yaw, *d_pitch, *d_duck, *d_out, *d_out2;
    void* ws;
    const int64_t ws_bytes = sdfr_workspace_bytes(&cam, N);
    CHECK(hipMalloc((void**)&d_origin, sizeof origin));
    CHECK(hipMalloc((void**)&d_yaw, sizeof yaw));
    CHECK(hipMalloc((void**)&d_pitch, sizeof pitch));
    CHECK(hipMalloc((void**)&d_duck, sizeof ducked));
    CHECK(hipMalloc((void**)&d_out, sizeof(float) * N * W * H));
    CHECK(hipMalloc((void**)&d_out2, sizeof(float) * N * W * H));
    CHECK(hipMalloc(&ws, (size_t)ws_bytes));
    CHECK(hipMemcpy(d_origin, origin, sizeof origin, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_yaw, yaw, sizeof yaw, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_pitch, pitch, sizeof pitch, hipMemcpyHostToDevice));
    CHECK(hipMemcpy(d_duck, ducked, sizeof ducked, hipMemcpyHostToDevice));

    SdfrPoses poses = {d_origin, 3, d_yaw, 1, d_pitch, 1, d_duck, 1, SDFR_F32, N};
    SdfrImage img = {d_out, (int64_t)W * H, SDFR_F32, 1, NULL};
    SdfrImage img2 = {d_out2, (int64_t)W * H, SDFR_F32, 1, NULL};
    if (sdfr_render(g, &cam, &poses, &img, ws, ws_bytes, NULL) != 0 ||
        sdfr_render_noalloc(g, &cam, &poses, &img2, NULL) != 0) {
        fprintf(stderr, "render: %s\n", sdfr_last_error());
        return 2;
    }
    /* a render the library must refuse: a workspace one byte short */
    if (sdfr_render(g, &cam, &poses, &img, ws, ws_bytes - 1, NULL) != -2 ||
        strstr(sdfr_last_error(), "workspace") == NULL) {
        fprintf(stderr, "a short workspace was not refused\n");
        return 1;
    }
    CHECK(hipDeviceSynchronize());
    float* got = (float*)malloc(sizeof(float) * N * W * H);
    float* got2 = (float*)malloc(sizeof(float) * N * W * H);
    float* want = (float*)malloc(sizeof(float) * N * W * H);
    CHECK(hipMemcpy(got, d_out, sizeof(float) * N * W * H, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(got2, d_out2, sizeof(float) * N * W * H, hipMemcpyDeviceToHost));
    if (oracle_render(grid, nx, ny, nz, mins, cell, W, H, 0, 120.0, 90.0, tan_h, tan_v, 1200.0f,
                      700.0f, 9.6f, 4.8f, 64, origin, yaw, pitch, ducked, N, want, NULL, NULL,
                      0) != 0) {
        fprintf(stderr, "oracle_render rejected its arguments\n");
        return 2;
    }
    int diff = 0, diff2 = 0, hits = 0;
    for (int i = 0; i < N * W * H; ++i) {
        diff += got[i] != want[i];
        diff2 += got2[i] != want[i];
        hits += want[i] < 0.5f;
    }
    printf("c-abi render: %d rays, %d differ from the oracle (noalloc: %d), %d hit within 350 u\n",
           N * W * H, diff, diff2, hits);
    sdfr_grid_destroy(g);
    return (diff || diff2 || hits == 0) ? 1 : 0;
}
