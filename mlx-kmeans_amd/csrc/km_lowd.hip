// Fused single-read pass for narrow rows (dims <= 16): exact assignment and per-cluster accumulation in one
// read of X, the job of the reference's fused and one-hot kernels (core.py:1478-1534, 1562-1675) for the
// low-d / large-n regime.
//
// Assignment. Each lane owns whole rows. Without the screen it runs the rows loop itself (core.py:263-274): for
// every centre in ascending order, s = sum_j (x_j - c_j)^2 with j ascending, product and add rounded separately,
// kept when s < best. With the screen (k >= 8) it first computes the expanded form a_c = |c|^2 - 2 x.c for every
// centre as a float32 FMA chain (d FMAs instead of the direct form's 3d operations), keeps the smallest and second
// smallest key (the centre index packed into the low mantissa bits), and proves with a rigorous error window that
// no other centre can hold the row's minimum; the direct form then runs on that one centre only. Rows the window
// cannot settle, and non-finite rows, run the full rows loop. Labels and best are the rows loop's, bit for bit,
// either way. Centres sit in LDS and are read by broadcast; each centre read serves the R rows a lane holds.
//
// Window. |fl(a_c) - A_c| <= E = gamma_{D+2} (max|c|^2 + 2 max|c| |x|) for every c (D FMA roundings over terms
// bounded by |c|^2 + 2 |x||c|, and |c|^2 itself rounded once from float64). The direct form s_c satisfies
// |s_c - D_c| <= g D_c (g = gamma_{D+2}), so a centre other than the screen's minimiser m can hold the minimum
// only if a_c - a_m <= 2E + 2 g/(1-g) D_m, with D_m <= |x|^2 + a_m + E; the packed index perturbs a key by at
// most RHO relative, which the test absorbs.
//
// Accumulation, deterministic by construction. A block is one wave. The wave keeps L = 64 >> lsh float32 tiles
// [count, best, x_0 .. x_{D-1}] x k clusters in LDS, laid out [cluster][column][L]: lane l adds its rows into
// column l % L, and the 64 / L lanes that share a column take turns in lane order (one pass per lane group, so
// each tile address has one writer per pass and the LDS executes the passes in program order). The L lanes of
// a pass touch L distinct consecutive columns: no bank conflicts. Every FOLD_ROWS additions per column the wave
// folds the tiles into float64 accumulators - each entry summed over the columns in a fixed rotation - and
// clears them, so no float32 accumulator ever adds more than FOLD_ROWS values (the reference adds 1024-row
// partials in plain float32 too, core.py:1562-1636). At the end the wave writes its float64 accumulators as one
// (sum, compensation) float32 pair per entry: the per-block partial that the fixed-order reduction reads. The
// plan picks the largest L whose LDS footprint still lets the register-limited number of waves reside: shared
// columns cost one LDS pass per lane group, private ones cost occupancy once k (d + 2) grows.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

template <int D, bool SCR>
struct LowGeo {
    static constexpr int W = D + 2;                                // columns: count, best, dims
    // rows per lane per iteration: the loads in flight while the previous rows are scored (the screen keeps the
    // shifted rows too, so above 4 dims it holds four rows to stay within three waves' registers)
    static constexpr int R = SCR ? (D <= 4 ? 8 : 4) : (D <= 8 ? 8 : 4);
    static constexpr int FOLD_ROWS = 256;                          // additions per tile column between folds
    static constexpr int FOLD_IT = FOLD_ROWS / R;                  // iterations between folds with private columns
};

__host__ __device__ constexpr size_t km_al16(size_t v) { return (v + 15) / 16 * 16; }

// LDS bytes of one block (one wave): centres, the 64 >> lsh tiles, the float64 accumulators, and with the
// screen the centres as [-2c, |c|^2] rows and once more dimension-major (the per-row gathers of one centre each)
__host__ __device__ inline size_t km_lowd_lds(int d, int k, bool screen, int lsh) {
    const size_t kw = (size_t)k * (d + 2);
    return km_al16((size_t)k * d * 4) + kw * (64 >> lsh) * 4 + kw * 8 +
           (screen ? km_al16((size_t)k * (d + 1) * 4) + km_al16((size_t)k * d * 4) : 0);
}

__host__ __device__ constexpr double km_lowd_gamma(int m) {
    return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08);
}

__device__ __forceinline__ float lowd_vmin(float a, float b) {
    float r;
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// a with its low index bits replaced by c: (mask & c) | (~mask & a) in one v_bfi_b32 (the mask in a VGPR, the
// wave-uniform index in an SGPR)
__device__ __forceinline__ float lowd_key(float a, uint32_t mask_v, uint32_t c) {
    float r;
    asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(mask_v), "s"(c), "v"(a));
    return r;
}
// v_min3_f32: two v_min_f32 in a row by definition (the same result for every input, NaN included)
__device__ __forceinline__ float lowd_vmin3(float a, float b, float c) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Largest k * (d + 2) served: the shared tiles (64 bytes per entry), the float64 accumulators (8) and the centres
// (under 8) stay within 64 KB of LDS.
static constexpr int KM_LOWD_MAX_KW = 768;
// Tile columns: 64 >> lsh, with 1 << lsh lanes taking turns on each (lsh = 0, 1, 2; the fold interval
// (256 / R) >> lsh stays at least one iteration for every R <= 16). Sharing costs one LDS read-modify-write pass
// per lane group and buys occupancy where the tiles, not the registers, limit it; the plan takes the least
// sharing that reaches the highest occupancy (measured on MI355X: 96M x 4, k = 12 with the screen: private 8
// waves per CU 465 us, two lanes per column 12 waves 417 us; 10M x 8, k = 8: 7 waves 90 us, 12 waves 85 us).
static constexpr int KM_LOWD_MAX_LSH = 2;

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

// F[e] += sum over the L columns of T[e], taken in the fixed rotation lane, lane+1, ... (mod L) so that lanes
// spread over the banks; then the tiles are cleared.
__device__ __forceinline__ void fold_tiles(float *T, double *F, int kw, int L, int lane) {
    wave_sync_lds();
    for (int e = lane; e < kw; e += 64) {
        const float *row = T + (size_t)e * L;
        double s = 0.0;
#pragma unroll 8
        for (int l = 0; l < L; l++) s += (double)row[(l + lane) & (L - 1)];
        F[e] += s;
    }
    wave_sync_lds();
    for (int e = lane; e < kw * L; e += 64) T[e] = 0.0f;
    wave_sync_lds();
}

template <int D, bool SCR, int LSH>
__global__ __launch_bounds__(64) void k_fused_lowd(const float *__restrict__ X, int64_t n,
                                                   const float *__restrict__ C, int k, int64_t rbs,
                                                   uint32_t *__restrict__ labels, float *__restrict__ best,
                                                   float *__restrict__ psum, float *__restrict__ pcomp, int rb0,
                                                   const int32_t *__restrict__ stop) {
    using G = LowGeo<D, SCR>;
    constexpr int W = G::W, R = G::R;
    // Window constants, in coordinates shifted by o (the centres' mean): x' = fl(x - o), c' = fl(c - o). The screen
    // a'_c = |c'|^2 - 2 x'.c' (FMA chain) is within E <= gE (|c'|^2 + 2 |x'||c'|) <= gE (2 max|c'|^2 + |x'|^2) of
    // |c~|^2 - 2 x~.c~ for the exact shifts x~ = x - o, c~ = c - o (D roundings of the chain, one of |c'|^2, and
    // the shifts' own roundings of at most u relative: gE = gamma_{D+5}), and D_c = |x~|^2 + |c~|^2 - 2 x~.c~. The
    // direct form is within gd = gamma_{D+2}/(1-gamma_{D+2}) relative. Margin = 2E + 2 gd (|x~|^2 + |a'_m| + E),
    // with |x~|^2 <= |x'|^2 (1 + 2 gamma_D + 4u), every coefficient inflated by 2^-18 for the float32 evaluation:
    // W_X |x'|^2 + W_A |a'_m| + w_c.
    constexpr double gE = km_lowd_gamma(D + 5), g2 = km_lowd_gamma(D + 2), gd = g2 / (1.0 - g2), up = 1.0 + 0x1p-18;
    constexpr float W_X = (float)((2.0 * gE + 2.0 * gd * (1.0 + gE)) * (1.0 + 2.0 * km_lowd_gamma(D) + 0x1p-22) * up);
    constexpr float W_A = (float)(2.0 * gd * up);
    constexpr float TINY = (float)((D + 2) * 0x1p-118);
    if (stop && *stop) return;
    extern __shared__ float lds[];
    const int lane = threadIdx.x;
    const int kw = k * W;
    constexpr int L = 64 >> LSH;                                          // tile columns
    constexpr int fold_it = G::FOLD_IT >> LSH;                            // 64 / L lanes add to each column
    float *Cl = lds;
    float *T = lds + km_al16((size_t)k * D * 4) / 4;                      // [kw][L]
    double *F = reinterpret_cast<double *>(T + (size_t)kw * L);           // [kw]
    float *Q = reinterpret_cast<float *>(F + kw);                         // [k][D + 1]: -2c, |c|^2 (screen)
    float *Ct = Q + km_al16((size_t)k * (D + 1) * 4) / 4;                // [D][k] (screen): lanes gathering
                                                                          // different centres hit different banks
    for (int e = lane; e < k * D; e += 64) Cl[e] = C[e];
    if constexpr (SCR)
        for (int e = lane; e < k * D; e += 64) Ct[(e % D) * k + e / D] = C[e];
    for (int e = lane; e < kw * L; e += 64) T[e] = 0.0f;
    for (int e = lane; e < kw; e += 64) F[e] = 0.0;
    // screen constants: the shift o, max |c'| (rounded up), max |c'|^2, and the index bits packed into keys
    float cnmax = 0.0f, csqmax = 0.0f;
    float o[D];
    int ib = 1;
    if constexpr (SCR) {
        wave_sync_lds();
#pragma unroll
        for (int j = 0; j < D; j++) {
            double t = 0.0;
            for (int c = 0; c < k; c++) t += (double)Cl[c * D + j];
            o[j] = (float)(t / k);
        }
        for (int c = lane; c < k; c += 64) {
            double sq = 0.0;
#pragma unroll
            for (int j = 0; j < D; j++) {
                const float v = C[c * D + j] - o[j];
                sq += (double)v * (double)v;
                Q[c * (D + 1) + j] = -2.0f * v;
            }
            const float sf = (float)sq;
            Q[c * (D + 1) + D] = sf;
            cnmax = fmaxf(cnmax, (float)(sqrt(sq) * (1.0 + 1e-6)));
            csqmax = fmaxf(csqmax, sf);
        }
        for (int off = 32; off > 0; off >>= 1) {
            cnmax = fmaxf(cnmax, __shfl_xor(cnmax, off));
            csqmax = fmaxf(csqmax, __shfl_xor(csqmax, off));
        }
        while ((1 << ib) < k) ib++;
    }
    const uint32_t imask = (1u << ib) - 1u;
    const uint32_t imask_v = __builtin_amdgcn_readfirstlane(imask);
    const float rho = (float)(1.01 * (double)(1 << ib) * 0x1p-23);
    const float csq2 = fmaxf(csqmax, cnmax * cnmax) * 2.0f * (1.0f + 0x1p-20f);
    const float w_c = (float)((2.0 * gE + 2.0 * gd * gE) * (1.0 + 0x1p-18)) * csq2 + 4.0f * TINY;

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
            if (r1 + STEP <= r_end) {   // the whole next step in range: one base address, constant offsets
                const float *xb = X + (r1 + lane) * D;
#pragma unroll
                for (int i = 0; i < R; i++) load_row<D>(xb + (int64_t)64 * D * i, 0, xn[i]);
            } else {
#pragma unroll
                for (int i = 0; i < R; i++) {
                    const int64_t row = r1 + 64 * i + lane;
                    load_row<D>(X, row < r_end ? row : r_end - 1, xn[i]);
                }
            }
        }
        float bst[R];
        uint32_t bl[R];
        if constexpr (SCR) {
            // the screen: smallest and second smallest packed key of |c'|^2 - 2 x'.c' per row
            float m1[R], m2[R], xs[R][D];
#pragma unroll
            for (int i = 0; i < R; i++) {
                m1[i] = 3.4e38f;
                m2[i] = 3.4e38f;
#pragma unroll
                for (int j = 0; j < D; j++) xs[i][j] = xr[i][j] - o[j];
            }
            // two centres at a time: the smallest of {m1, m2, a, b} is min3(m1, a, b) (m1 <= m2), the second the
            // smaller of m2 and the middle of (m1, a, b)
            int c = 0;
            for (; c + 1 < k; c += 2) {
                float q[D + 1], p[D + 1];
#pragma unroll
                for (int j = 0; j <= D; j++) {
                    q[j] = Q[c * (D + 1) + j];
                    p[j] = Q[(c + 1) * (D + 1) + j];
                }
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float a = q[D], b = p[D];
#pragma unroll
                    for (int j = 0; j < D; j++) {
                        a = __builtin_fmaf(xs[i][j], q[j], a);
                        b = __builtin_fmaf(xs[i][j], p[j], b);
                    }
                    const float ka = lowd_key(a, imask_v, (uint32_t)c);
                    const float kb = lowd_key(b, imask_v, (uint32_t)(c + 1));
                    m2[i] = lowd_vmin(m2[i], __builtin_amdgcn_fmed3f(m1[i], ka, kb));
                    m1[i] = lowd_vmin3(m1[i], ka, kb);
                }
            }
            if (c < k) {
                float q[D + 1];
#pragma unroll
                for (int j = 0; j <= D; j++) q[j] = Q[c * (D + 1) + j];
#pragma unroll
                for (int i = 0; i < R; i++) {
                    float a = q[D];
#pragma unroll
                    for (int j = 0; j < D; j++) a = __builtin_fmaf(xs[i][j], q[j], a);
                    const float key = lowd_key(a, imask_v, (uint32_t)c);
                    m2[i] = __builtin_amdgcn_fmed3f(m1[i], m2[i], key);
                    m1[i] = lowd_vmin(m1[i], key);
                }
            }
            bool full[R];
#pragma unroll
            for (int i = 0; i < R; i++) {
                float xsq = 0.0f;
#pragma unroll
                for (int j = 0; j < D; j++) xsq = __builtin_fmaf(xs[i][j], xs[i][j], xsq);
                const float km = m1[i];
                const float akm = __builtin_fmaf(rho, fabsf(km), km);
                // margin 2E + 2 GDIR D_m with E <= GAM (max|c|^2 + max|c|^2 + |x|^2) (2ab <= a^2 + b^2) and
                // D_m <= |x|^2 + |a_m| + E: linear in |x|^2 and |a_m|, constants folded on the host side of it
                const float margin = __builtin_fmaf(W_X, xsq, __builtin_fmaf(W_A, fabsf(akm), w_c));
                float Tw = akm + margin;
                Tw = __builtin_fmaf(0x1p-22f, fabsf(Tw), Tw);
                const uint32_t cm = __float_as_uint(km) & imask;
                const uint32_t cmc = cm < (uint32_t)k ? cm : 0u;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < D; j++) {
                    const float t = xr[i][j] - Ct[j * k + cmc];
                    s = s + t * t;
                }
                // settled: no second centre inside the window, a finite row (xsq) and distance, an index below k
                const bool settled = __builtin_fmaf(-rho, fabsf(m2[i]), m2[i]) > Tw && xsq < INFINITY &&
                                     s < INFINITY && cm < (uint32_t)k;
                full[i] = !settled;
                bst[i] = s;
                bl[i] = cmc;
            }
            // Rows the window leaves open run the rows loop with the whole wave: the row is broadcast, every lane
            // scores its centres (lane, lane + 64, ...) in the direct form, and the wave keeps the smallest
            // distance, the lowest index among equal ones - the rows loop's result, including label 0 and best
            // +inf when no distance is below +inf.
#pragma unroll
            for (int i = 0; i < R; i++) {
                uint64_t need = __ballot(full[i]);
                while (need) {
                    const int L = __builtin_ctzll(need);
                    need &= need - 1;
                    float xb[D];
#pragma unroll
                    for (int j = 0; j < D; j++)
                        xb[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xr[i][j]), L));
                    float bv = INFINITY;
                    uint32_t bi = 0;
                    for (int c = lane; c < k; c += 64) {
                        float sc = 0.0f;
#pragma unroll
                        for (int j = 0; j < D; j++) {
                            const float t = xb[j] - Ct[j * k + c];
                            sc = sc + t * t;
                        }
                        if (sc < bv) {
                            bv = sc;
                            bi = (uint32_t)c;
                        }
                    }
#pragma unroll
                    for (int off = 32; off > 0; off >>= 1) {
                        const float ov = __shfl_xor(bv, off);
                        const uint32_t oi = (uint32_t)__shfl_xor((int)bi, off);
                        if (ov < bv || (ov == bv && oi < bi)) {
                            bv = ov;
                            bi = oi;
                        }
                    }
                    if (lane == L) {
                        bst[i] = bv;
                        bl[i] = bi;
                    }
                }
            }
        } else {
            // the rows loop for R rows at once
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
        }
        // outputs, then each row into this lane's tile column, one lane group after another
#pragma unroll
        for (int i = 0; i < R; i++) {
            const int64_t row = r0 + 64 * i + lane;
            if (row < r_end) {
                if (labels) labels[row] = bl[i];
                if (best) best[row] = bst[i];
            }
        }
        const int grp = lane / L;
#pragma unroll
        for (int g = 0; g < (1 << LSH); g++) {
            if (LSH == 0 || grp == g) {
#pragma unroll
                for (int i = 0; i < R; i++) {
                    const int64_t row = r0 + 64 * i + lane;
                    if (row < r_end) {
                        float *t = T + (size_t)bl[i] * (W * L) + (lane % L);
                        t[0] += 1.0f;
                        t[L] += bst[i];
#pragma unroll
                        for (int j = 0; j < D; j++) t[(2 + j) * L] += xr[i][j];
                    }
                }
            }
        }
        if (++it == fold_it) {
            it = 0;
            fold_tiles(T, F, kw, L, lane);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < R; i++)
#pragma unroll
                for (int j = 0; j < D; j++) xr[i][j] = xn[i][j];
        }
    }
    if (it) fold_tiles(T, F, kw, L, lane);
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

#define KM_LOWD_FNS(S, H)                                                                                     \
    {nullptr,                k_fused_lowd<1, S, H>,  k_fused_lowd<2, S, H>,  k_fused_lowd<3, S, H>,              \
     k_fused_lowd<4, S, H>,  k_fused_lowd<5, S, H>,  k_fused_lowd<6, S, H>,  k_fused_lowd<7, S, H>,              \
     k_fused_lowd<8, S, H>,  k_fused_lowd<9, S, H>,  k_fused_lowd<10, S, H>, k_fused_lowd<11, S, H>,             \
     k_fused_lowd<12, S, H>, k_fused_lowd<13, S, H>, k_fused_lowd<14, S, H>, k_fused_lowd<15, S, H>,             \
     k_fused_lowd<16, S, H>}
// [screen][lsh][dims]
static lowd_fn g_lowd[2][KM_LOWD_MAX_LSH + 1][17] = {
    {KM_LOWD_FNS(false, 0), KM_LOWD_FNS(false, 1), KM_LOWD_FNS(false, 2)},
    {KM_LOWD_FNS(true, 0), KM_LOWD_FNS(true, 1), KM_LOWD_FNS(true, 2)}};
#undef KM_LOWD_FNS

static int lowd_rows_per_iter(int d, bool scr) { return 64 * (scr ? (d <= 4 ? 8 : 4) : (d <= 8 ? 8 : 4)); }

// The screen costs d + 2.5 operations per centre and row against the direct form's 3d + 3, plus a per-row window
// and one direct form with an LDS gather; measured on MI355X it is the faster of the two from about 8 centres on
// (96M x 4, k = 12: 465 against 471 us private, 417 with shared columns; 10M x 8, k = 8: 85 against 90 us).
static bool lowd_screen(int k) { return k >= 8; }

km_lowd_plan km_plan_lowd(const km_device_info &dev, int64_t n, int d, int k, bool aligned, int64_t max_blocks) {
    km_lowd_plan pl{};
    if (d < 1 || d > 16 || k < 1 || n < 1) return pl;
    if ((int64_t)k * (d + 2) > KM_LOWD_MAX_KW) return pl;
    if ((d % 2 == 0) && !aligned) return pl;   // vector row loads need 8/16-byte aligned rows
    const bool scr = lowd_screen(k);
    // the least column sharing that reaches the highest occupancy
    int lsh = -1, occ = 0;
    for (int h = 0; h <= KM_LOWD_MAX_LSH; h++) {
        const size_t b = km_lowd_lds(d, k, scr, h);
        int o = 0;
        if (b > 65536 || hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, (const void *)g_lowd[scr][h][d], 64, b) !=
                             hipSuccess)
            o = 0;
        if (o > occ) {
            occ = o;
            lsh = h;
        }
    }
    if (occ < 1) return pl;
    const size_t lds = km_lowd_lds(d, k, scr, lsh);
    const int64_t unit = lowd_rows_per_iter(d, scr);
    const int64_t units = (n + unit - 1) / unit;
    int64_t nrb = (int64_t)dev.cus * occ;
    if (nrb > units) nrb = units;
    if (max_blocks > 0 && nrb > max_blocks) nrb = max_blocks;
    if (nrb < 1) nrb = 1;
    int64_t rbs = (n + nrb - 1) / nrb;
    rbs = (rbs + unit - 1) / unit * unit;
    pl.ok = 1;
    pl.screen = scr ? 1 : 0;
    pl.rbs = rbs;
    pl.nrb = (int)((n + rbs - 1) / rbs);
    pl.lds = lds;
    pl.lsh = lsh;
    return pl;
}

hipError_t km_launch_lowd(const km_lowd_plan &pl, const float *X, int64_t n, int d, const float *C, int k,
                          uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, const int32_t *stop,
                          hipStream_t s) {
    if (!pl.ok || d < 1 || d > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(g_lowd[pl.screen ? 1 : 0][pl.lsh][d], dim3(pl.nrb), dim3(64), pl.lds, s, X, n, C, k,
                       pl.rbs, labels, best, psum, pcomp, rb0, stop);
    return hipGetLastError();
}
