// Fused single-read pass for narrow rows (dims <= 16): exact assignment and per-cluster accumulation in one
// read of X, the job of the reference's fused and one-hot kernels (core.py:1478-1534, 1562-1675) for the
// low-d / large-n regime.
//
// Assignment. Each lane owns whole rows and runs the rows loop itself (core.py:263-274): for every centre in
// ascending order, s = sum_j (x_j - c_j)^2 with j ascending, product and add rounded separately, kept when
// s < best. Labels and best are therefore the rows loop's, bit for bit. Centres sit in LDS and are read by
// broadcast; each centre read serves the R rows a lane holds.
//
// Accumulation, deterministic by construction. A block is one wave. Every lane has a private float32 tile
// [count, best, x_0 .. x_{D-1}] x k clusters in LDS, laid out [cluster][column][lane]: a lane adds its row
// into its own column of addresses (one LDS bank per lane, so no conflicts and no shared address), in row
// order. Every FOLD_ROWS rows per lane the wave folds the 64 tiles into float64 accumulators - each entry summed
// over the lanes in a fixed rotation - and clears them, so no float32 accumulator ever adds more than
// FOLD_ROWS values (the reference adds 1024-row partials in plain float32 too, core.py:1562-1636). At the end
// the wave writes its float64 accumulators as one (sum, compensation) float32 pair per entry: the per-block
// partial that the fixed-order reduction reads.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

template <int D>
struct LowGeo {
    static constexpr int W = D + 2;                                // columns: count, best, dims
    static constexpr int R = D <= 4 ? 8 : D <= 8 ? 4 : 2;          // rows per lane per iteration
    static constexpr int FOLD_ROWS = 256;                          // rows per lane between float64 folds
    static constexpr int FOLD_IT = FOLD_ROWS / R;                  // iterations between folds
};

__host__ __device__ constexpr size_t km_al16(size_t v) { return (v + 15) / 16 * 16; }

// LDS bytes of one block (one wave): centres, the 64 lane tiles, the float64 accumulators
__host__ __device__ inline size_t km_lowd_lds(int d, int k) {
    const size_t kw = (size_t)k * (d + 2);
    return km_al16((size_t)k * d * 4) + kw * 64 * 4 + kw * 8;
}

// Largest k * (d + 2) served: the tiles take 256 bytes per entry.
static constexpr int KM_LOWD_MAX_KW = 224;

template <int D>
__device__ __forceinline__ void load_row(const float *__restrict__ X, int64_t row, float (&x)[D]) {
    if constexpr (D % 4 == 0) {
        const float4 *p = reinterpret_cast<const float4 *>(X + row * D);
#pragma unroll
        for (int q = 0; q < D / 4; q++) {
            const float4 v = p[q];
            x[4 * q] = v.x;
            x[4 * q + 1] = v.y;
            x[4 * q + 2] = v.z;
            x[4 * q + 3] = v.w;
        }
    } else if constexpr (D % 2 == 0) {
        const float2 *p = reinterpret_cast<const float2 *>(X + row * D);
#pragma unroll
        for (int q = 0; q < D / 2; q++) {
            const float2 v = p[q];
            x[2 * q] = v.x;
            x[2 * q + 1] = v.y;
        }
    } else {
#pragma unroll
        for (int j = 0; j < D; j++) x[j] = X[row * D + j];
    }
}

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// F[e] += sum over lanes of T[e][lane], lanes taken in the fixed rotation lane, lane+1, ... (mod 64) so the 64
// lanes read 64 distinct banks; then the tiles are cleared.
__device__ __forceinline__ void fold_tiles(float *T, double *F, int kw, int lane) {
    wave_sync_lds();
    for (int e = lane; e < kw; e += 64) {
        const float *row = T + (size_t)e * 64;
        double s = 0.0;
#pragma unroll 8
        for (int l = 0; l < 64; l++) s += (double)row[(l + lane) & 63];
        F[e] += s;
    }
    wave_sync_lds();
    for (int e = lane; e < kw * 64; e += 64) T[e] = 0.0f;
    wave_sync_lds();
}

template <int D>
__global__ __launch_bounds__(64) void k_fused_lowd(const float *__restrict__ X, int64_t n,
                                                   const float *__restrict__ C, int k, int64_t rbs,
                                                   uint32_t *__restrict__ labels, float *__restrict__ best,
                                                   float *__restrict__ psum, float *__restrict__ pcomp, int rb0,
                                                   const int32_t *__restrict__ stop) {
    using G = LowGeo<D>;
    constexpr int W = G::W, R = G::R;
    if (stop && *stop) return;
    extern __shared__ float lds[];
    const int lane = threadIdx.x;
    const int kw = k * W;
    float *Cl = lds;
    float *T = lds + km_al16((size_t)k * D * 4) / 4;                      // [kw][64]
    double *F = reinterpret_cast<double *>(T + (size_t)kw * 64);          // [kw]

    for (int e = lane; e < k * D; e += 64) Cl[e] = C[e];
    for (int e = lane; e < kw * 64; e += 64) T[e] = 0.0f;
    for (int e = lane; e < kw; e += 64) F[e] = 0.0;

    const int64_t r_begin = (int64_t)blockIdx.x * rbs;
    const int64_t r_end = (r_begin + rbs < n) ? r_begin + rbs : n;
    constexpr int64_t STEP = (int64_t)64 * R;

    float xr[R][D];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int64_t row = r_begin + 64 * i + lane;
        load_row<D>(X, row < r_end ? row : r_end - 1, xr[i]);
    }
    wave_sync_lds();

    int it = 0;
    for (int64_t r0 = r_begin; r0 < r_end; r0 += STEP) {
        // prefetch the next iteration's rows (wave-uniform condition)
        float xn[R][D];
        const int64_t r1 = r0 + STEP;
        const bool more = r1 < r_end;
        if (more) {
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int64_t row = r1 + 64 * i + lane;
                load_row<D>(X, row < r_end ? row : r_end - 1, xn[i]);
            }
        }
        // the rows loop for R rows at once
        float bst[R];
        uint32_t bl[R];
#pragma unroll
        for (int i = 0; i < R; i++) {
            bst[i] = INFINITY;
            bl[i] = 0;
        }
        for (int c = 0; c < k; c++) {
            float cc[D];
#pragma unroll
            for (int j = 0; j < D; j++) cc[j] = Cl[c * D + j];
#pragma unroll
            for (int i = 0; i < R; i++) {
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < D; j++) {
                    const float t = xr[i][j] - cc[j];
                    s = s + t * t;
                }
                if (s < bst[i]) {
                    bst[i] = s;
                    bl[i] = (uint32_t)c;
                }
            }
        }
        // outputs, then each row into this lane's tile
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int64_t row = r0 + 64 * i + lane;
            if (row < r_end) {
                if (labels) labels[row] = bl[i];
                if (best) best[row] = bst[i];
                float *t = T + (size_t)bl[i] * (W * 64) + lane;
                t[0] += 1.0f;
                t[64] += bst[i];
#pragma unroll
                for (int j = 0; j < D; j++) t[(2 + j) * 64] += xr[i][j];
            }
        }
        if (++it == G::FOLD_IT) {
            it = 0;
            fold_tiles(T, F, kw, lane);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int j = 0; j < D; j++) xr[i][j] = xn[i][j];
        }
    }
    if (it) fold_tiles(T, F, kw, lane);
    // this block's partial as a float32 (sum, compensation) pair per entry
    float *ps = psum + (int64_t)(rb0 + blockIdx.x) * kw;
    float *pc = pcomp + (int64_t)(rb0 + blockIdx.x) * kw;
    for (int e = lane; e < kw; e += 64) {
        const double t = F[e];
        const float hi = (float)t;
        ps[e] = hi;
        pc[e] = (float)(t - (double)hi);
    }
}

// ------------------------------------------------------------------ planning and launch

typedef void (*lowd_fn)(const float *, int64_t, const float *, int, int64_t, uint32_t *, float *, float *, float *,
                        int, const int32_t *);

static lowd_fn g_lowd[17] = {nullptr,          k_fused_lowd<1>,  k_fused_lowd<2>,  k_fused_lowd<3>,
                             k_fused_lowd<4>,  k_fused_lowd<5>,  k_fused_lowd<6>,  k_fused_lowd<7>,
                             k_fused_lowd<8>,  k_fused_lowd<9>,  k_fused_lowd<10>, k_fused_lowd<11>,
                             k_fused_lowd<12>, k_fused_lowd<13>, k_fused_lowd<14>, k_fused_lowd<15>,
                             k_fused_lowd<16>};

static int g_lowd_cus = 0;

static int lowd_rows_per_iter(int d) { return 64 * (d <= 4 ? 8 : d <= 8 ? 4 : 2); }

km_lowd_plan km_plan_lowd(int64_t n, int d, int k, bool aligned) {
    km_lowd_plan pl{};
    if (d < 1 || d > 16 || k < 1 || n < 1) return pl;
    if ((int64_t)k * (d + 2) > KM_LOWD_MAX_KW) return pl;
    if ((d % 2 == 0) && !aligned) return pl;   // vector row loads need 8/16-byte aligned rows
    const size_t lds = km_lowd_lds(d, k);
    if (g_lowd_cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            g_lowd_cus = prop.multiProcessorCount;
        if (g_lowd_cus <= 0) g_lowd_cus = 256;
    }
    if (lds > 65536) return pl;
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)g_lowd[d], 64, lds) != hipSuccess ||
        occ < 1)
        occ = 1;
    const int64_t unit = lowd_rows_per_iter(d);
    const int64_t units = (n + unit - 1) / unit;
    int64_t nrb = (int64_t)g_lowd_cus * occ;
    if (nrb > units) nrb = units;
    if (nrb < 1) nrb = 1;
    int64_t rbs = (n + nrb - 1) / nrb;
    rbs = (rbs + unit - 1) / unit * unit;
    pl.ok = 1;
    pl.rbs = rbs;
    pl.nrb = (int)((n + rbs - 1) / rbs);
    pl.lds = lds;
    return pl;
}

hipError_t km_launch_lowd(const km_lowd_plan &pl, const float *X, int64_t n, int d, const float *C, int k,
                          uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, const int32_t *stop,
                          hipStream_t s) {
    if (!pl.ok || d < 1 || d > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(g_lowd[d], dim3(pl.nrb), dim3(64), pl.lds, s, X, n, C, k, pl.rbs, labels, best, psum,
                       pcomp, rb0, stop);
    return hipGetLastError();
}
