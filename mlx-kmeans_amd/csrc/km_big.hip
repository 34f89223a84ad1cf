// Exact Lloyd pass for wide rows (16 < dims <= 1536, k <= 65536): the reference's "tiles" design (core.py:616-651,
// 310-377: matrix-unit dot products, an error margin, exact rescoring of the candidates) rebuilt for CDNA4, plus
// its sorted accumulation (core.py:934-994, 424-449, 1421-1441).
//
//   k_big_rows      once per dataset: the rows as bf16 MFMA B operands, X16T[tile][K-step][lane][8] (coalesced
//                   1 KB per wave per K-step), and |x|^2 rounded up per row
//   k_big_centres   per pass: the centres as bf16 MFMA A operands, Cop[chunk][K-step][lane][8], with one extra
//                   K-step carrying |c|^2 against a B operand of ones; |c| (rounded up) and |c|^2 per centre
//   k_big_screen    a'_c = |c|^2 - 2 x.c for every (row, centre) on the matrix cores, never stored, in one pass
//                   over the centres: the row's smallest packed key (value, centre index) so far, and the centres
//                   inside the error window around it - every centre that can hold the exact minimum
//   k_big_rescore   the rows loop (core.py:263-274) on those candidates only, ascending index, strict '<'
//   k_big_fullscan  rows whose window holds more centres of one half-row than its list takes (16; 32 above 768
//                   dims) or non-finite data: every centre, 64 rows x 64 centres per block step; without a row
//                   list, every row of a part (the rows loop's tiled form, km_launch_rows_tiled)
//   k_big_hist/scan/scatter   a stable counting sort of the rows by label; then the per-cluster float64 sums in
//                   row order, in fixed chunks of sorted rows (km_chunks.hip): the totals of the pass
//
// Labels and best are the rows loop's bit for bit (see the window below). With mode KM_APPROX the screen's
// minimiser is taken on trust, as the reference's exact=False path does (core.py:878-890, 1061-1088), only its
// distance is computed exactly.
//
// Large k (more than 4096 centres, the regime the reference's cascade pruning serves, core.py:1091-1260): the keys
// carry no index (PACK = false; no perturbation either), each listed key keeps its centre index beside it in LDS,
// the counting sort keeps its counters in global memory, and exact=False is served exactly.
#pragma clang fp contract(off)
#include "km_internal.h"
#include "kmeans_hip.h"
#include <math.h>

#include <algorithm>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float kb_f4 __attribute__((ext_vector_type(4)));
typedef unsigned int kb_u4 __attribute__((ext_vector_type(4)));

// candidates a half-row's list holds: 16, and 32 above 48 K-steps (769 dims and wider, where a row's window crowds
// more centres; one screen block per CU leaves the LDS for it). The global lists hold 2 kb_list_half(DS) slots per
// row, the half-rows' lists at slots 0 and kb_list_half(DS).
__host__ __device__ constexpr int kb_list_half(int DS) { return DS > 48 ? 32 : 16; }
static constexpr int KB_LIST_MAX = 32;    // the longest half-row list
static constexpr int KB_SLICE = 25;       // most A-operand K-steps per LDS slice (1 KB each): 768 dims take two
                                          // slices per chunk, so two block barriers and a prefetch of half a chunk
// Above 48 K-steps one block per CU has the LDS to itself: slices of up to 49 K-steps, two per chunk (500k x 960 /
// 1536, k = 1024, us per screen: 25-step slices 1721 / 2224, 49-step slices 1636 / 2205)
static constexpr int KB_SLICE_WIDE = 49;
__host__ __device__ constexpr int kb_slice(int ds) { return ds > 48 ? KB_SLICE_WIDE : KB_SLICE; }
static constexpr int KB_WAVES = 4;        // waves per screen block (32 rows each)
// A-fragment K-steps in flight above 48 K-steps, where one wave per SIMD has no other wave to cover the LDS
// latency (500k x 960 / 1536, k = 1024, us per screen: 3 steps 1795 / 2318, 6 steps 1720 / 2262, 9 steps 1726 / 2232)
static constexpr int KB_PF_WIDE = 9;
static constexpr int KB_OVER = 0xffff;    // ncand value: scan every centre
static constexpr double KB_APPROX_LIMIT = 65504.0 / 4;   // the reference's APPROX_FP16_LIMIT (core.py:1035)

__host__ __device__ constexpr double kb_gamma(int m) {
    return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08);
}

__device__ __forceinline__ uint32_t kb_u32(float v) { return __float_as_uint(v); }
__device__ __forceinline__ float kb_f32(uint32_t v) { return __uint_as_float(v); }
__device__ __forceinline__ float kb_min(float a, float b) {
    float r;
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// v_min3_f32: two v_min_f32 in a row by definition (the same result for every input, NaN included)
__device__ __forceinline__ float kb_min3(float a, float b, float c) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// value of lane l ^ 32
__device__ __forceinline__ float kb_partner(float v, int lane) {
    const auto r = __builtin_amdgcn_permlane32_swap(kb_u32(v), kb_u32(v), false, false);
    return kb_f32(lane < 32 ? r[1] : r[0]);
}
__device__ __forceinline__ float kb_u32f(uint32_t v) { return __uint_as_float(v); }
__device__ __forceinline__ uint32_t kb_f32u(float v) { return __float_as_uint(v); }

// ------------------------------------------------------------------ rows (once per dataset)

// Thread per (tile, K-step, lane): 8 bf16 of row 32 tile + (lane & 31), dims 16 s + 8 (lane >> 5) + q.
__global__ __launch_bounds__(256) void k_big_rows(const float *__restrict__ X, int64_t n, int d, int DS,
                                                  uint16_t *__restrict__ X16T, int64_t ntiles) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= ntiles * DS * 64) return;
    const int lane = (int)(e & 63);
    const int64_t ts = e >> 6;
    const int s = (int)(ts % DS);
    const int64_t tile = ts / DS;
    const int64_t row = tile * 32 + (lane & 31);
    const int j0 = 16 * s + 8 * (lane >> 5);
    uint32_t w[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        float a = 0.0f, b = 0.0f;
        if (row < n) {
            if (j0 + 2 * p < d) a = X[row * d + j0 + 2 * p];
            if (j0 + 2 * p + 1 < d) b = X[row * d + j0 + 2 * p + 1];
        }
        const __bf16 ha = (__bf16)a, hb = (__bf16)b;
        w[p] = (uint32_t)(*reinterpret_cast<const uint16_t *>(&ha)) |
               ((uint32_t)(*reinterpret_cast<const uint16_t *>(&hb)) << 16);
    }
    *reinterpret_cast<uint4 *>(X16T + e * 8) = make_uint4(w[0], w[1], w[2], w[3]);
}

// Wave per row: xn[2 row] = |x|^2 and xn[2 row + 1] = |bf16(x) - x| (the norm of the screen operand's rounding
// residual), float64 sums (dims split over lanes, fixed butterfly) rounded up into float32; +inf when the row is
// not finite.
__global__ __launch_bounds__(256) void k_big_xsq(const float *__restrict__ X, int64_t n, int d,
                                                 float *__restrict__ xn) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    double s = 0.0, r = 0.0;
    bool fin = true;
    for (int j = lane; j < d; j += 64) {
        const float v = X[row * d + j];
        fin = fin && isfinite(v);
        s += (double)v * (double)v;
        const double e = (double)(float)(__bf16)v - (double)v;
        r += e * e;
    }
    for (int off = 32; off > 0; off >>= 1) {
        s += __shfl_xor(s, off);
        r += __shfl_xor(r, off);
    }
    const bool all = __all(fin);
    if (lane == 0) {
        const bool ok = all && s * (1.0 + 0x1p-20) < 3.0e38;
        xn[2 * row] = ok ? (float)(s * (1.0 + 0x1p-20)) : INFINITY;
        xn[2 * row + 1] = ok ? (float)(sqrt(r) * (1.0 + 0x1p-20)) : INFINITY;
    }
}

// The largest |x|^2 of a slice (float bits of the non-negative xn[2 row], +inf included) into *xmax by an
// integer maximum: for non-negative floats the bit patterns order as the values do.
__global__ __launch_bounds__(256) void k_big_xmax(const float *__restrict__ xn, int64_t n, uint32_t *__restrict__ xmax) {
    uint32_t m = 0;
    for (int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x; r < n; r += (int64_t)gridDim.x * 256)
        m = max(m, kb_u32(xn[2 * r]));
    for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
    if ((threadIdx.x & 63) == 0) atomicMax(xmax, m);
}

// ------------------------------------------------------------------ centres (per pass)

// Wave per centre: |c|^2 (float64 sum of the float32 values, dims ascending within each lane then a fixed
// butterfly), |c| rounded up, and |bf16(-2c) + 2c| (the operand's rounding residual) rounded up in cn[kpad + c].
// Padding centres (k <= c < kpad): csq = 3e38 (never a candidate), cn = 0.
__global__ __launch_bounds__(256) void k_big_cnorm(const float *__restrict__ C, int k, int kpad, int d,
                                                   float *__restrict__ csq, float *__restrict__ cn,
                                                   km_control *__restrict__ ctl, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    if (blockIdx.x == 0 && threadIdx.x == 0) {   // rows the next screen lists for a full scan / a rescoring
        ctl->n_over = 0;
        ctl->n_multi = 0;
    }
    const int c = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (c >= kpad) return;
    double s = 0.0, r = 0.0;
    if (c < k)
        for (int j = lane; j < d; j += 64) {
            const float v = C[(int64_t)c * d + j];
            s += (double)v * (double)v;
            const float m2 = -2.0f * v;
            const double e = (double)(float)(__bf16)m2 - (double)m2;
            r += e * e;
        }
    for (int off = 32; off > 0; off >>= 1) {
        s += __shfl_xor(s, off);
        r += __shfl_xor(r, off);
    }
    if (lane == 0) {
        csq[c] = c < k ? (float)s : 3.0e38f;
        cn[c] = c < k ? (float)(sqrt(s) * (1.0 + 1e-6)) : 0.0f;
        cn[kpad + c] = c < k ? (float)(sqrt(r) * (1.0 + 1e-6)) : 0.0f;
    }
}

// Thread per (chunk, K-step, lane): Cop for K-step s < DS holds bf16(-2 c[32 chunk + (lane & 31)][16 s + 8 h + q]);
// K-step DS holds |c|^2 as two bf16 pieces in q = 0, 1 of the h = 0 lanes. One block also writes
// maxes = {max |c| (rounded up), max |c|^2, max |bf16(-2c) + 2c|} over the real centres.
__global__ __launch_bounds__(256) void k_big_centres(const float *__restrict__ C, int k, int d, int DS, int nchunks,
                                                     const float *__restrict__ csq, const float *__restrict__ cn,
                                                     uint16_t *__restrict__ Cop, float *__restrict__ maxes,
                                                     const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int AK = DS + 1;
    if (e < (int64_t)nchunks * AK * 64) {
        const int lane = (int)(e & 63);
        const int64_t cs = e >> 6;
        const int s = (int)(cs % AK);
        const int ch = (int)(cs / AK);
        const int c = 32 * ch + (lane & 31);
        const int h = lane >> 5;
        uint16_t out[8];
        for (int q = 0; q < 8; q++) {
            float v = 0.0f;
            if (s < DS) {
                const int j = 16 * s + 8 * h + q;
                if (c < k && j < d) v = -2.0f * C[(int64_t)c * d + j];
            } else if (h == 0 && q < 2) {
                const float sf = csq[c];
                const float hi = (float)(__bf16)sf;
                v = q == 0 ? hi : sf - hi;
            }
            const __bf16 b = (__bf16)v;
            out[q] = *reinterpret_cast<const uint16_t *>(&b);
        }
        *reinterpret_cast<uint4 *>(Cop + e * 8) = *reinterpret_cast<const uint4 *>(out);
    }
    if (blockIdx.x == 0) {
        __shared__ float a[256], b[256], r[256];
        const int kpad = nchunks * 32;
        float mn = 0.0f, ms = 0.0f, mr = 0.0f;
        for (int c = threadIdx.x; c < k; c += 256) {
            mn = fmaxf(mn, cn[c]);
            ms = fmaxf(ms, csq[c]);
            mr = fmaxf(mr, cn[kpad + c]);
        }
        a[threadIdx.x] = mn;
        b[threadIdx.x] = ms;
        r[threadIdx.x] = mr;
        __syncthreads();
        for (int h = 128; h > 0; h >>= 1) {
            if ((int)threadIdx.x < h) {
                a[threadIdx.x] = fmaxf(a[threadIdx.x], a[threadIdx.x + h]);
                b[threadIdx.x] = fmaxf(b[threadIdx.x], b[threadIdx.x + h]);
                r[threadIdx.x] = fmaxf(r[threadIdx.x], r[threadIdx.x + h]);
            }
            __syncthreads();
        }
        if (threadIdx.x == 0) {
            maxes[0] = a[0];
            maxes[1] = b[0];
            maxes[2] = r[0];
        }
    }
}

// ------------------------------------------------------------------ the screen
//
// Window. For a row x and centre c, A_c = |c|^2 - 2 x.c and D_c = |x - c|^2 = |x|^2 + A_c (exact reals). The
// matrix cores give a'_c = sum_j bf16(x_j) bf16(-2 c_j) + q_h + q_l (|c|^2 as two bf16 pieces). With the rounding
// residuals e = bf16(x) - x and f_c = bf16(-2c) - (-2c) (their norms computed exactly per row and per centre and
// rounded up), sum_j bf16(x_j) bf16(-2c_j) + 2 x.c = -2 e.c + x.f_c + e.f_c, so by Cauchy-Schwarz its size is at
// most 2|e||c| + |x||f_c| + |e||f_c|. Products of bf16 values are exact in float32; the float32 accumulation of
// NACC = DP + 2 terms adds at most gamma_NACC times their absolute sum (<= 2.04 |x||c| + 1.01 |c|^2); the
// two-piece |c|^2 is off by at most 2^-16 relative. Hence, uniformly in c,
//     |a'_c - A_c| <= E = (2|e| max|c| + |x| max|f| + |e| max|f|)(1 + 2^-20) + 2.04 gamma_NACC |x| max|c|
//                         + GAM2 max|c|^2 + FLUSH (|x| + max|c|) + TINY,     GAM2 = 1.01 gamma_NACC + 2^-16 + 2^-23
// (bf16 rounding to nearest has unit roundoff 2^-8, so |e| <= 2^-8 |x| and |f| <= 2^-7 |c|: E is never above the
// plain worst case, and for typical data it is about 2.5 times smaller). The rows loop's float32 direct form s_c satisfies |s_c - D_c| <= g D_c (g = gamma_{D+2}), so a
// centre can hold the minimum only if a'_c - a'_m <= 2E + 2 g/(1-g) D_m, with D_m <= |x|^2 + a'_m + E for the
// screen minimiser m. Keys carry the centre index in their low IB mantissa bits (relative perturbation <= RHO),
// absorbed by the test. The window only narrows as the row's smallest key falls, so the screen lists, chunk by
// chunk, every centre inside the window of the smallest key seen so far, prunes a full list against the current
// window, and at the end keeps the listed centres inside the final window - exactly the centres the final window
// admits. A half-row with more than kb_list_half(DS) of them at once (16 up to 768 dims, 32 above), or non-finite
// data, sends the row to a full scan.

// The window's error bound E for a row (see above) with DS K-steps, from its |x|^2 (rounded up), |bf16(x) - x| and
// the centres' maxes {max |c|, max |c|^2, max |f|}; nx gets |x| rounded up.
template <int DS>
__device__ __forceinline__ float kb_screen_E(float xsq_up, float exn, const float *__restrict__ maxes, float &nx) {
    constexpr km_screen_k q = km_screen_consts(16 * DS + 2);
    return km_screen_E(xsq_up, exn, maxes[0], maxes[1], maxes[2], q, nx);
}

// The per-centre bounds from screen values: D_c >= |x|^2 + a'_c - E. With |x|^2 >= xsq_up (1 - 2^-18) and every
// |a'_c| at most max|c|^2 + 2 |x| max|c| + E, the slack 2^-21 (|x|^2 + E + max |a'|) covers the float32 additions,
// so lbase + a'_c (as computed) is at most D_c.
__device__ __forceinline__ float kb_lbase(float xsq_up, float E, float nx, const float *__restrict__ maxes) {
    const float xlo = xsq_up * (1.0f - 0x1p-18f);
    const float amax = maxes[1] + 2.0f * nx * maxes[0] + E;
    return (xlo - E) - 0x1p-21f * (xlo + E + amax);
}

// The wave's 32 rows stay in registers as B operands (4 per K-step): up to 48 K-steps two blocks share a CU (256
// registers a wave); above that one block does, and the 512 registers of a lone wave per SIMD (accumulation
// registers included, which the matrix cores read operands from) hold up to 96 K-steps without spilling.
// What the bound-writing instance writes besides the screen's own outputs (the per-centre bounds between passes,
// km_bounds.hip): per row ub / ubl (an upper bound, hi-scaled, on the distance to the screen minimiser, and that
// centre), and with wlb this tile's float16 lower bounds sqrt(|x|^2 + a'_c - E) lo, rounded toward zero.
struct kb_bnd_out {
    uint16_t *lb;
    float *ub;
    uint32_t *ubl;
    float lo, hi;
    bool lists;   // also the candidate lists (a tile the plain screen does not take this pass)
    float *sraw;        // plain instance: the sample tiles' raw screen values (null: none)
    int64_t sstride;    // ... of the tiles t with t % sstride == 0
};

// One 32-row tile per wave (tile >= ntiles: a wave of zero rows that only takes part in the block's barriers).
template <int DS, bool PACK, bool BND>
__device__ __forceinline__ void kb_screen_tile(
    int64_t tile, const uint16_t *__restrict__ X16T, const float *__restrict__ xsq, int64_t n, int d,
    const uint16_t *__restrict__ Cop, const float *__restrict__ maxes, int k, int nchunks, int ib, float rho,
    int approx, uint16_t *__restrict__ ncand, uint16_t *__restrict__ cand, uint32_t *__restrict__ over,
    uint32_t *__restrict__ multi, km_control *__restrict__ ctl, const kb_bnd_out &bnd) {
    constexpr int LH = kb_list_half(DS);   // this width's list length per half-row
    constexpr int DP = 16 * DS, AK = DS + 1;
    constexpr float TINY = (float)((DP + 2) * 0x1p-118);
    extern __shared__ float lds[];
    char *ring = reinterpret_cast<char *>(lds);   // two slices of at most kb_slice(DS) K-steps, 1 KB each
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int h = lane >> 5;
    const int64_t ntiles = (n + 31) / 32;
    const bool have = tile < ntiles;
    const int64_t row = tile * 32 + (lane & 31);
    const bool real_row = have && row < n;

    // this wave's 32 rows as B operands (zeros past the last tile)
    bf16x8 B[DS];
#pragma unroll
    for (int s = 0; s < DS; s++) {
        if (have) {   // each row once per pass: non-temporal
            const kb_u4 q = __builtin_nontemporal_load(reinterpret_cast<const kb_u4 *>(X16T + ((tile * DS + s) * 64 + lane) * 8));
            const uint4 v = make_uint4(q.x, q.y, q.z, q.w);
            B[s] = *reinterpret_cast<const bf16x8 *>(&v);
        } else {
            B[s] = bf16x8{};
        }
    }
    bf16x8 Bone;
#pragma unroll
    for (int q = 0; q < 8; q++) Bone[q] = (__bf16)((h == 0 && q < 2) ? 1.0f : 0.0f);
    const uint32_t IMASK = PACK ? (1u << ib) - 1u : 0u;
    // up to 48 K-steps (two waves per SIMD) ~IMASK is held in a vector register, so that packing a key is one
    // v_and_or_b32 with the index in a scalar register (768 dims: 1.58 -> 1.54 ms per screen); a lone wave per SIMD
    // does better with the compiler's v_and + v_or3 (1536 dims: 3.45 ms against 3.51)
    uint32_t nmask = ~IMASK;
    if constexpr (DS <= 48) asm("v_mov_b32 %0, %1" : "=v"(nmask) : "s"(~IMASK));
    if (!PACK) approx = 0;

    // A operand slices: chunk ch is SPC slices of SLK K-steps (the last possibly shorter), staged through a
    // two-slice LDS ring; slice g is loaded while slice g - 1 is multiplied.
    constexpr int SPC = (AK + kb_slice(DS) - 1) / kb_slice(DS);
    constexpr int SLK = (AK + SPC - 1) / SPC;
    const int GP = nchunks * SPC;
    const int G = GP;
    auto issue = [&](int g) {
        char *buf = ring + (g & 1) * (SLK * 1024);
        const int gl = g % GP;
        const int ch = gl / SPC, sl = gl - (gl / SPC) * SPC;
        const int s0 = sl * SLK;
        const int ns = (AK - s0) < SLK ? (AK - s0) : SLK;
        for (int j = wave; j < ns; j += KB_WAVES) {
            // the K-step's base is wave-uniform: kept in scalar registers (the saddr form of the load), so the
            // ring costs one lane-offset VGPR instead of a 64-bit address per slice
            const uint64_t bse = (uint64_t)(uintptr_t)(Cop + ((int64_t)ch * AK + s0 + j) * 64 * 8);
            const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)bse);
            const uint32_t bhi = __builtin_amdgcn_readfirstlane((uint32_t)(bse >> 32));
            const uint16_t *src = (const uint16_t *)(uintptr_t)(((uint64_t)bhi << 32) | blo) + lane * 8;
            __builtin_amdgcn_global_load_lds((gbl_vptr)src, (lds_vptr)(buf + j * 1024), 16, 0, 0);
        }
    };
    // one chunk's screen values: acc element v is centre 32 ch + 8 (v / 4) + 4 h + v % 4 against this lane's row
    auto screen_chunk = [&](int g0, f32x16 &acc) {
        acc = f32x16{};
#pragma unroll
        for (int sl = 0; sl < SPC; sl++) {
            const int g = g0 + sl;
            const char *cur = ring + (g & 1) * (SLK * 1024);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (g + 1 < G) issue(g + 1);
            // A fragments PF K-steps ahead of their MFMA (PF + 1 register sets in rotation), the reads and MFMAs
            // interleaved one for one: the LDS latency is covered by PF MFMAs
            constexpr int PF = DS > 48 ? KB_PF_WIDE : 3;
            bf16x8 Ab[PF + 1];
#pragma unroll
            for (int j = 0; j < PF; j++)
                if (sl * SLK + j < AK && j < SLK) Ab[j] = *reinterpret_cast<const bf16x8 *>(cur + j * 1024 + lane * 16);
#pragma unroll
            for (int j = 0; j < SLK; j++) {
                const int s = sl * SLK + j;   // compile-time after unrolling
                if (j + PF < SLK && s + PF < AK)
                    Ab[(j + PF) % (PF + 1)] = *reinterpret_cast<const bf16x8 *>(cur + (j + PF) * 1024 + lane * 16);
                if (s < AK)
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Ab[j % (PF + 1)], s < DS ? B[s < DS ? s : 0] : Bone,
                                                                   acc, 0, 0, 0);
            }
            // the chunk's last slice may hold fewer K-steps (LAST): its groups are counted from its own length
            constexpr int LAST = AK - (SPC - 1) * SLK, PFL = PF < LAST ? PF : LAST;
            if (sl + 1 < SPC || LAST == SLK) {
                __builtin_amdgcn_sched_group_barrier(0x100, PF, 0);   // PF LDS reads,
#pragma unroll
                for (int j = 0; j < SLK - PF; j++) {                    // then MFMA, LDS read, ...,
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, PF, 0);   // and the last PF MFMAs
            } else {
                __builtin_amdgcn_sched_group_barrier(0x100, PFL, 0);
#pragma unroll
                for (int j = 0; j < LAST - PFL; j++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, PFL, 0);
            }
        }
    };

    const float xsq_up = real_row ? xsq[2 * row] : 0.0f;
    const float exn = real_row ? xsq[2 * row + 1] : 0.0f;
    // per-row window terms: T(m) = a + margin(a), a = m + rho |m|, for the row's smallest key m so far. T only
    // falls as m falls, so a centre kept against an earlier T is a superset of those the final T admits.
    const float GDIR = (float)(kb_gamma(d + 2) / (1.0 - kb_gamma(d + 2)) * (1.0 + 0x1p-20));
    float nx;
    const float E = kb_screen_E<DS>(xsq_up, exn, maxes, nx);
    const float lbase = BND ? kb_lbase(xsq_up, E, nx, maxes) : 0.0f;   // the bound-writing instance's
    // a key bound Tp with key <= Tp whenever key - rho |key| <= T
    auto key_bound = [&](float m) {
        const float akm = m + rho * fabsf(m);
        const float dm_up = fmaxf(0.0f, xsq_up + akm + E) * (1.0f + 0x1p-20f);
        float T = akm + ((2.0f * E + 2.0f * GDIR * dm_up) * (1.0f + 0x1p-20f) + TINY);
        T = T + 0x1p-22f * fabsf(T);
        float Tp = (T >= 0.0f ? T / (1.0f - rho) : T / (1.0f + rho));
        Tp = Tp + 0x1p-21f * fabsf(Tp);
        return (T < INFINITY) ? Tp : -INFINITY;
    };
    // One pass over the centre chunks. Per chunk: the row's smallest key so far (both halves), its key bound, and
    // this chunk's keys inside it appended to this lane's list in LDS (up to LH; a full list is first pruned
    // against the current bound, and if still full the row takes the full scan). Approximate mode keeps only the
    // smallest key.
    // LH slots per lane and one more that takes the fast path's writes of keys outside the window
    float *list = reinterpret_cast<float *>(ring + 2 * SLK * 1024) + (size_t)wave * (LH + 1) * 64 + lane;
    // without packed keys, the listed keys' centre indices (after the KB_WAVES lists of keys)
    uint16_t *lidx = reinterpret_cast<uint16_t *>(reinterpret_cast<float *>(ring + 2 * SLK * 1024) +
                                                  (size_t)KB_WAVES * (LH + 1) * 64) +
                     (size_t)wave * (LH + 1) * 64 + lane;
    // a sample tile of the per-centre bounds (32-bit arithmetic: a slice has fewer than 2^27 tiles)
    const bool sample = !BND && bnd.sraw && have && (uint32_t)tile % (uint32_t)bnd.sstride == 0u;
    float *sdst = sample ? bnd.sraw + ((int64_t)((uint32_t)tile / (uint32_t)bnd.sstride) * nchunks * 64 + lane) * 16
                         : nullptr;
    issue(0);
    float m1 = 3.4e38f;
    int cnt = 0;
    bool spill = false;
    for (int ch = 0; ch < nchunks; ch++) {
        f32x16 acc;
        screen_chunk(ch * SPC, acc);
        float key[16], cmin = 0.0f;   // this chunk's smallest key
#pragma unroll
        for (int v = 0; v < 16; v++) {
            // the packed index leaves out the half-row's own bit (4 h: bit 2 of every centre index), so it is the
            // same in every lane; the list a key sits in, or the winning half-row, puts it back
            uint32_t cidx = (uint32_t)(32 * ch + 8 * (v >> 2) + (v & 3));
            if constexpr (DS <= 48) asm("s_or_b32 %0, %1, %2" : "=s"(cidx) : "s"(32 * ch), "n"(8 * (v >> 2) + (v & 3)));
            key[v] = PACK ? kb_f32((kb_u32(acc[v]) & nmask) | cidx) : acc[v];
            // Without packing, key[v] is the matrix cores' result register itself: the first instruction to
            // read it must be compiled code, whose hazard tracking inserts the wait states an MFMA result needs
            // (inline assembly here read stale accumulators); packed keys go through v_min3 in pairs
            if (!PACK) cmin = v == 0 ? key[0] : fminf(cmin, key[v]);
            else if (v == 1) cmin = kb_min(key[0], key[1]);
            else if (v >= 3 && (v & 1)) cmin = kb_min3(cmin, key[v - 1], key[v]);
        }
        m1 = PACK ? kb_min(m1, cmin) : fminf(m1, cmin);
        if (!BND && sample) {   // a sample tile: its raw values, 64 B per lane
            float4 *dst = reinterpret_cast<float4 *>(sdst + (int64_t)ch * 1024);
            dst[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
            dst[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
            dst[2] = make_float4(acc[8], acc[9], acc[10], acc[11]);
            dst[3] = make_float4(acc[12], acc[13], acc[14], acc[15]);
        }
        if (BND && have) {   // this chunk's lower bounds, 32 contiguous bytes per lane
            uint32_t pk[8];
#pragma unroll
            for (int v = 0; v < 16; v += 2) {
                const float a0 = fminf(__builtin_sqrtf(fmaxf(lbase + acc[v], 0.0f)) * bnd.lo, 65504.0f);
                const float a1 = fminf(__builtin_sqrtf(fmaxf(lbase + acc[v + 1], 0.0f)) * bnd.lo, 65504.0f);
                pk[v / 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a0, a1));
            }
            uint4 *dst = reinterpret_cast<uint4 *>(bnd.lb + ((tile * nchunks + ch) * 64 + lane) * 16);
            dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        }
        if (approx) continue;
        const float mrow = kb_min(m1, kb_partner(m1, lane));
        const float Tp = key_bound(mrow);
        // a key inside the window somewhere in the wave: this chunk's smallest one is (a NaN key is never inside)
        if (__ballot(cmin <= Tp)) {
            // a lane whose list overflowed takes no more keys (its row takes the full scan): its bound is -inf
            const float Tl = spill ? -INFINITY : Tp;
            int nin = 0;   // this lane's keys to be listed
#pragma unroll
            for (int v = 0; v < 16; v++) nin += key[v] <= Tl ? 1 : 0;
            if (!__ballot(cnt + nin > LH)) {
                // no lane's list fills up with a key still to come: every key is written at the lane's next slot
                // (at most the spare slot past the list, where a full or overflowed list stands) and counted only
                // when it is listed
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    if (!PACK) lidx[cnt * 64] = (uint16_t)(32 * ch + 8 * (v >> 2) + 4 * h + (v & 3));
                    list[cnt * 64] = key[v];
                    cnt += key[v] <= Tl ? 1 : 0;
                }
            } else {
            uint64_t bal[16];
#pragma unroll
            for (int v = 0; v < 16; v++) bal[v] = __ballot(key[v] <= Tp);
#pragma unroll
            for (int v = 0; v < 16; v++) {
                if ((bal[v] >> lane) & 1ull) {
                    if (cnt == LH && !spill) {   // full: drop what the current bound already excludes
                        int w = 0;
                        for (int q = 0; q < LH; q++) {
                            const float kq = list[q * 64];
                            if (kq <= Tp) {
                                if (!PACK) lidx[w * 64] = lidx[q * 64];
                                list[(w++) * 64] = kq;
                            }
                        }
                        cnt = w;
                        spill = cnt == LH;
                    }
                    if (cnt < LH) {
                        if (!PACK) lidx[cnt * 64] = (uint16_t)(32 * ch + 8 * (v >> 2) + 4 * h + (v & 3));
                        list[(cnt++) * 64] = key[v];
                    }
                }
            }
            }
        }
    }
    // both halves of the row: the smaller key, half-row 0's on a tie (its centre index is the lower); hbit is the
    // winning half-row's bit 2 of the minimiser's centre index
    const float m1o = kb_partner(m1, lane);
    const bool other = m1o < m1 || (m1o == m1 && h == 1) || (m1 != m1 && m1o == m1o);
    const uint32_t hbit = (uint32_t)(other ? h ^ 1 : h) << 2;
    m1 = kb_min(m1, m1o);
    const bool finite = xsq_up < INFINITY && m1 < 3.0e38f;
    if (!approx && finite && real_row) {
        // the final bound: keep the listed centres inside it
        const float Tp = key_bound(m1);
        int w = 0;
        for (int q = 0; q < cnt; q++) {
            const float kq = list[q * 64];
            if (kq <= Tp && (!BND || bnd.lists))
                cand[row * (2 * LH) + h * LH + (w++)] = PACK ? (uint16_t)((kb_u32(kq) & IMASK) | (uint32_t)(4 * h))
                                                            : lidx[q * 64];
        }
        cnt = w;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (!real_row) return;
    // The other half-row's count, or LH + 1 when its list overflowed: a lane's count never exceeds LH
    // (the final filter only lowers it), so the overflow has to travel as its own value.
    const int cnt_o = (int)kb_f32u(kb_partner(kb_u32f((uint32_t)(spill ? LH + 1 : cnt)), lane));
    const bool spill_o = cnt_o > LH;
    if (h != 0) return;
    if (BND) {   // an upper bound on the distance to the minimiser m (D_m <= |x|^2 + a'_m + E), and m
        float u = INFINITY;
        if (finite) {
            const float dm_up = fmaxf(0.0f, xsq_up + (m1 + rho * fabsf(m1)) + E) * (1.0f + 0x1p-20f);
            u = __builtin_sqrtf(dm_up) * bnd.hi;
        }
        bnd.ub[row] = u < INFINITY ? u : INFINITY;
        bnd.ubl[row] = (kb_u32(m1) & IMASK) | hbit;
        if (!bnd.lists) return;
    }
    int code;
    if (!finite) {
        code = KB_OVER;   // non-finite data: the rows loop decides
    } else if (approx) {
        cand[row * (2 * LH)] = (uint16_t)((kb_u32(m1) & IMASK) | hbit);
        code = 1;
    } else if (spill || spill_o || cnt + cnt_o == 0) {
        code = KB_OVER;   // an empty window cannot happen for finite data (the minimiser is inside it)
    } else {
        code = cnt | (cnt_o << 8);
    }
    ncand[row] = (uint16_t)code;
    if (code == KB_OVER) over[atomicAdd(&ctl->n_over, 1u)] = (uint32_t)row;
    // rows with several candidates: one counter update per wave, each row at its place among the wave's
    const bool is_multi = code != KB_OVER && (code & 255) + (code >> 8) >= 2;
    const uint64_t mm = __ballot(is_multi);
    if (mm) {
        const int leader = __ffsll((unsigned long long)mm) - 1;
        uint32_t base = 0;
        if (lane == leader) base = atomicAdd(&ctl->n_multi, (uint32_t)__popcll(mm));
        base = (uint32_t)__shfl((int)base, leader);
        if (is_multi) multi[base + (uint32_t)__popcll(mm & ((1ull << lane) - 1ull))] = (uint32_t)row;
    }
}

template <int DS, bool PACK>
__global__ __launch_bounds__(64 * KB_WAVES, DS > 48 ? 1 : 2) void k_big_screen(
    const uint16_t *__restrict__ X16T, const float *__restrict__ xsq, int64_t n, int d,
    const uint16_t *__restrict__ Cop, const float *__restrict__ maxes, int k, int nchunks, int ib, float rho,
    int approx, const uint32_t *__restrict__ xmax, uint16_t *__restrict__ ncand, uint16_t *__restrict__ cand,
    uint32_t *__restrict__ over, uint32_t *__restrict__ multi, km_control *__restrict__ ctl,
    const int32_t *__restrict__ stop, float *__restrict__ sraw, int64_t sstride) {
    if (stop && *stop) return;
    // Approximate mode only while this pass's centres pass the reference's half-precision guard (core.py:1055-1058):
    // sqrt(max |x|^2 max |c|^2) < 65504 / 4, from the data's largest |x|^2 (rounded up, +inf if any row is not
    // finite) and the largest |c|^2 of the centres. Otherwise the pass is exact.
    if (approx) approx = sqrt((double)kb_f32(*xmax) * (double)maxes[1]) < KB_APPROX_LIMIT;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kb_bnd_out out{};
    out.sraw = sraw;
    out.sstride = sstride;
    kb_screen_tile<DS, PACK, false>((int64_t)blockIdx.x * KB_WAVES + wave, X16T, xsq, n, d, Cop, maxes, k, nchunks,
                                    ib, rho, approx, ncand, cand, over, multi, ctl, out);
}

// The screen of a pass that builds the per-centre bounds (packed keys): every tile's lists, as the plain screen
// writes them, plus its float16 bounds and every row's ub. A grid of one round of blocks loops over the tiles (on
// the passes that do not build, the launch costs only its blocks' start).
template <int DS>
__global__ __launch_bounds__(64 * KB_WAVES, DS > 48 ? 1 : 2) void k_big_screen_bnd(
    const uint16_t *__restrict__ X16T, const float *__restrict__ xsq, int64_t n, int d,
    const uint16_t *__restrict__ Cop, const float *__restrict__ maxes, int k, int nchunks, int ib, float rho,
    uint16_t *__restrict__ ncand, uint16_t *__restrict__ cand, uint32_t *__restrict__ over,
    uint32_t *__restrict__ multi, km_control *__restrict__ ctl, uint16_t *__restrict__ lb, float *__restrict__ ub,
    uint32_t *__restrict__ ubl, float lo, float hi, const km_bnd *__restrict__ bs) {
    if (bs->skip_bscreen) return;
    const int64_t ntiles = (n + 31) / 32;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const kb_bnd_out out{lb, ub, ubl, lo, hi, true, nullptr, 1};
    for (int64_t wb = blockIdx.x; wb * KB_WAVES < ntiles; wb += gridDim.x) {   // block-uniform
        __syncthreads();   // every wave is done with the previous tile's A slices before the ring is refilled
        kb_screen_tile<DS, true, true>(wb * KB_WAVES + wave, X16T, xsq, n, d, Cop, maxes, k, nchunks, ib, rho, 0,
                                       ncand, cand, over, multi, ctl, out);
    }
}

// ------------------------------------------------------------------ exact rescoring

// One wave (a block of 64 threads) per KB_RR consecutive rows. Each (row, candidate) pair is a work item, items
// ordered by row and then by ascending candidate index (each row's lane sorts its own list); a lane takes one item
// per round. KB_SCH dims at a time, the wave stages its rows and its items' centres in LDS (coalesced loads, stride
// KB_SCH + 1 floats so lanes on different rows or items read different banks), the next chunk's loads in flight in
// registers while the current chunk is used; every item carries its running direct-form sum across the chunks, so
// the dims are added in ascending order. Then one lane per row takes its items in order with a strict '<': the
// rows loop restricted to the candidates. The wave shares its LDS with no other wave, so ordering its own LDS
// accesses takes no block barrier. Rows marked KB_OVER are left to k_big_fullscan. With LITE (passes that return
// no per-row distances) the waves take KB_RR entries at a time of the screen's list of rows with several
// candidates; single-candidate rows take their label in k_big_label1, and the sorted accumulation adds the
// distances.
static constexpr int KB_RR = 16;      // rows per rescoring wave
static constexpr int KB_RT = 64;      // lanes (= items per round) per rescoring wave
static constexpr int KB_RCH = 32;     // dims per LDS chunk (the full scan's)
static constexpr int KB_SCH = 32;     // dims per LDS chunk of the rescoring
static constexpr int KB_SLN = KB_SCH / 4;        // lanes staging one row's (or item's) chunk as float4s
static constexpr int KB_SRW = KB_RT / KB_SLN;    // rows (items) one staging step covers
static constexpr int KB_RITEMS = KB_RR * 2 * KB_LIST_MAX;   // items of one wave's rows at most

// orders this wave's LDS accesses: every lane's earlier reads and writes before any later one
__device__ __forceinline__ void kb_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <bool V4, bool LITE>
__global__ __launch_bounds__(KB_RT) void k_big_rescore(const float *__restrict__ X, int64_t n, int d,
                                                       const float *__restrict__ C, int k,
                                                       const uint16_t *__restrict__ ncand,
                                                       const uint16_t *__restrict__ cand, int slot,
                                                       const uint32_t *__restrict__ list,
                                                       const km_control *__restrict__ ctl,
                                                       uint32_t *__restrict__ labels, float *__restrict__ best,
                                                       const int32_t *__restrict__ stop, km_bnd_refresh bref) {
    if (stop && *stop) return;
    // with per-centre bounds that describe every tile: each item's exact distance refreshes its bound, and each
    // row's result its upper bound (wave-uniform)
    const bool refresh = bref.lb && bref.bs->built;
    __shared__ uint32_t rid[KB_RR];   // the wave's rows: consecutive, or entries of the list
    __shared__ float xs[KB_RR * (KB_SCH + 1)];
    __shared__ float cs[KB_RT * (KB_SCH + 1)];
    __shared__ uint16_t it_c[KB_RITEMS];
    __shared__ uint8_t it_r[KB_RITEMS];
    __shared__ float it_s[KB_RITEMS];
    const int lane = threadIdx.x;
    const int64_t total = LITE ? (int64_t)ctl->n_multi : n;
    for (int64_t r0 = (int64_t)blockIdx.x * KB_RR; r0 < total; r0 += (int64_t)gridDim.x * KB_RR) {
    const int nr = (int)((total - r0) < KB_RR ? (total - r0) : KB_RR);
    kb_wave_sync();   // the previous rows' LDS is no longer read
    // item lists: lane r owns row r; an inclusive scan of the counts gives each row its slots
    int code = KB_OVER, cntr = 0;
    uint32_t myrow = 0;
    if (lane < nr) {
        myrow = LITE ? list[r0 + lane] : (uint32_t)(r0 + lane);
        rid[lane] = myrow;
        code = ncand[myrow];
        cntr = code == KB_OVER ? 0 : (code & 255) + (code >> 8);
    }
    int incl = cntr;
    for (int off = 1; off < KB_RR; off <<= 1) {
        const int v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
    }
    const int items = __shfl(incl, KB_RR - 1);   // lanes past nr count nothing
    const int b = incl - cntr;
    if (lane < nr && cntr > 0) {
        int m = b;
        for (int half = 0; half < 2; half++) {
            const int nc = half ? code >> 8 : code & 255;
            for (int i = 0; i < nc; i++) {
                const uint16_t v = cand[(int64_t)myrow * (2 * slot) + half * slot + i];
                int j = m - 1;
                while (j >= b && it_c[j] > v) { it_c[j + 1] = it_c[j]; j--; }
                it_c[j + 1] = v;
                it_r[m] = (uint8_t)lane;
                m++;
            }
        }
    }
    kb_wave_sync();
    // staging: with V4 (dims a multiple of 4, rows 16-byte aligned) KB_SLN consecutive lanes fetch one
    // KB_SCH-float chunk as float4s - lane t takes float4 t % KB_SLN of rows and of items t / KB_SLN + KB_SRW u;
    // otherwise floats
    constexpr int XPT = KB_RR * KB_SCH / KB_RT;   // x values staged per lane per chunk
    constexpr int CPT = KB_SCH;                   // centre values staged per lane per chunk (KB_RT items)
    for (int q0 = 0; q0 < items; q0 += KB_RT) {
        const int ni = (items - q0) < KB_RT ? (items - q0) : KB_RT;
        const int q = q0 + lane;
        const int ir = q < items ? (int)it_r[q] : 0;
        float sacc = 0.0f;
        float xv[XPT], cv[CPT];
        const float *cbase[CPT / 4];
        if (V4) {
#pragma unroll
            for (int u = 0; u < CPT / 4; u++) {
                const int i = lane / KB_SLN + KB_SRW * u;
                cbase[u] = i < ni ? C + (int64_t)it_c[q0 + i] * d + 4 * (lane % KB_SLN) : nullptr;
            }
        }
        auto fetch = [&](int j0) {
            const int w = (d - j0) < KB_SCH ? (d - j0) : KB_SCH;
            if (V4) {
#pragma unroll
                for (int u = 0; u < XPT / 4; u++) {
                    const int r = lane / KB_SLN + KB_SRW * u, p = lane % KB_SLN;
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (r < nr && 4 * p < w) {   // each listed row once per pass: non-temporal
                        const kb_f4 qv = __builtin_nontemporal_load(reinterpret_cast<const kb_f4 *>(X + (int64_t)rid[r] * d + j0 + 4 * p));
                        v = make_float4(qv.x, qv.y, qv.z, qv.w);
                    }
                    xv[4 * u] = v.x;
                    xv[4 * u + 1] = v.y;
                    xv[4 * u + 2] = v.z;
                    xv[4 * u + 3] = v.w;
                }
#pragma unroll
                for (int u = 0; u < CPT / 4; u++) {
                    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (cbase[u] && 4 * (lane % KB_SLN) < w) v = *reinterpret_cast<const float4 *>(cbase[u] + j0);
                    cv[4 * u] = v.x;
                    cv[4 * u + 1] = v.y;
                    cv[4 * u + 2] = v.z;
                    cv[4 * u + 3] = v.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < XPT; u++) {
                    const int e = lane + KB_RT * u;
                    const int r = e / KB_SCH, jj = e % KB_SCH;
                    xv[u] = (r < nr && jj < w) ? X[(int64_t)rid[r] * d + j0 + jj] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < CPT; u++) {
                    const int e = lane + KB_RT * u;
                    const int i = e / KB_SCH, jj = e % KB_SCH;
                    cv[u] = (i < ni && jj < w) ? C[(int64_t)it_c[q0 + i] * d + j0 + jj] : 0.0f;
                }
            }
        };
        fetch(0);
        for (int j0 = 0; j0 < d; j0 += KB_SCH) {
            const int w = (d - j0) < KB_SCH ? (d - j0) : KB_SCH;
            kb_wave_sync();   // the previous chunk's LDS is no longer read
            if (V4) {
#pragma unroll
                for (int u = 0; u < XPT; u++)
                    xs[(lane / KB_SLN + KB_SRW * (u / 4)) * (KB_SCH + 1) + 4 * (lane % KB_SLN) + (u % 4)] = xv[u];
#pragma unroll
                for (int u = 0; u < CPT; u++)
                    cs[(lane / KB_SLN + KB_SRW * (u / 4)) * (KB_SCH + 1) + 4 * (lane % KB_SLN) + (u % 4)] = cv[u];
            } else {
#pragma unroll
                for (int u = 0; u < XPT; u++) {
                    const int e = lane + KB_RT * u;
                    xs[(e / KB_SCH) * (KB_SCH + 1) + e % KB_SCH] = xv[u];
                }
#pragma unroll
                for (int u = 0; u < CPT; u++) {
                    const int e = lane + KB_RT * u;
                    cs[(e / KB_SCH) * (KB_SCH + 1) + e % KB_SCH] = cv[u];
                }
            }
            kb_wave_sync();
            if (j0 + KB_SCH < d) fetch(j0 + KB_SCH);
            if (q < items) {
                const float *xr = xs + ir * (KB_SCH + 1);
                const float *cc = cs + lane * (KB_SCH + 1);
                float sv = sacc;
                // a whole chunk unrolled: its LDS reads issue ahead of the dependent sum (dims still ascending)
                if (w == KB_SCH) {
#pragma unroll
                    for (int jj = 0; jj < KB_SCH; jj++) {
                        const float t = xr[jj] - cc[jj];
                        sv = sv + t * t;
                    }
                } else {
                    for (int jj = 0; jj < w; jj++) {
                        const float t = xr[jj] - cc[jj];
                        sv = sv + t * t;
                    }
                }
                sacc = sv;
            }
        }
        if (q < items) it_s[q] = sacc;
    }
    kb_wave_sync();
    if (lane < nr && code != KB_OVER) {
        float bst = INFINITY;
        uint32_t bl = 0;
        for (int q = b; q < b + cntr; q++) {
            const float sq = it_s[q];
            if (sq < bst) { bst = sq; bl = (uint32_t)it_c[q]; }
        }
        labels[myrow] = bl;
        best[myrow] = bst;
        if (refresh) {
            const float u = (bst >= 0.0f && bst < INFINITY) ? __builtin_sqrtf(bst) * bref.hi : INFINITY;
            bref.ub[myrow] = u < INFINITY ? u : INFINITY;
            bref.ubl[myrow] = bl;
        }
    }
    if (refresh) {
        // lb_c = sqrt(s_c) lo + S_c (frame), rounded toward zero: s_c <= D_c (1 + g), so sqrt(s_c) lo is at most
        // sqrt(D_c) (1 - g); 1 - 2^-22 covers the float32 addition. A non-finite distance or drift writes 0.
        for (int q = lane; q < items; q += KB_RT) {
            const int64_t r = rid[it_r[q]];
            const int c = it_c[q];
            const float sq = it_s[q], sc = bref.S[c];
            float v = 0.0f;
            if (sc < INFINITY && sq >= 0.0f)
                v = sq < INFINITY ? fminf((__builtin_sqrtf(sq) * bref.lo + sc) * (1.0f - 0x1p-22f), 65504.0f) : 65504.0f;
            const uint32_t hv = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(v, 0.0f));
            bref.lb[km_bnd_index(r, c, bref.nchunks)] = (uint16_t)hv;
        }
    }
    }
}

// Labels of the rows whose window held a single candidate (passes without per-row distances; the rescoring
// takes the listed rows with several).
__global__ __launch_bounds__(256) void k_big_label1(const uint16_t *__restrict__ ncand, const uint16_t *__restrict__ cand,
                                                    int64_t n, int slot, uint32_t *__restrict__ labels,
                                                    const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (r >= n) return;
    const int code = ncand[r];
    if (code != KB_OVER && (code & 255) + (code >> 8) == 1) labels[r] = cand[r * (2 * slot) + ((code & 255) ? 0 : slot)];
}

// Rows the screen could not narrow (more than kb_list_half window centres in a half-row, or non-finite data) take the
// rows loop over every centre. Blocks of 256 threads take 64 listed rows at a time against chunks of 64 centres:
// 32 dims of the rows and of the centres staged in LDS per step, each thread carrying 4 rows x 4 centres of
// direct-form sums (dims ascending, product and add rounded separately) across the steps, then keeping per row
// the smallest distance with a strict '<' over its centres in ascending order. The 16 threads that share a row
// then reduce (value, index) with the lowest index on ties: the rows loop's label and best, label 0 and best +inf
// included when no distance compares below +inf.
// Above KB_FSPLIT centres the centres are split into ranges of KB_FSPLIT, one block per (tile, range), so that a
// handful of listed rows still spreads over the chip. Each range's result (value, index) goes into the row's 64-bit
// key by an atomic minimum of (value bits << 32 | index): distances are non-negative or NaN, NaN is never taken
// (strict '<'), so the key order is the value order and then the index order - the smallest distance, the lowest
// index among equal ones, whatever order the ranges finish in. The key starts at (+inf, 0).
// Without a list (over null) the kernel is the rows loop for all n_direct rows of a part, tile t holding rows
// 64 t ..: the assignment of rows wider than the screen serves, whose rows fit no thread's registers.
static constexpr int KB_FR = 64;        // rows per full-scan tile
static constexpr int KB_FC = 64;        // centres per full-scan chunk
static constexpr int KB_FSPLIT = 256;   // centres per range of the split full scan
static constexpr uint64_t KB_FKEY0 = (uint64_t)0x7f800000u << 32;   // (+inf, label 0)
__global__ __launch_bounds__(256) void k_big_fullscan(const float *__restrict__ X, int d, const float *__restrict__ C,
                                                      int k, const uint32_t *__restrict__ over, int64_t n_direct,
                                                      km_control *__restrict__ ctl, uint32_t *__restrict__ labels,
                                                      float *__restrict__ best, uint64_t *__restrict__ keys,
                                                      const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    __shared__ float xs[KB_RCH][KB_FR + 1];   // [dim][row]
    __shared__ float cs[KB_RCH][KB_FC + 1];   // [dim][centre]
    __shared__ int64_t rows[KB_FR];
    const int tid = threadIdx.x;
    const int tr = tid >> 4, tc = tid & 15;   // rows 4 tr .. 4 tr + 3, centres 4 tc .. 4 tc + 3 of a chunk
    const uint32_t total = over ? ctl->n_over : (uint32_t)n_direct;
    if (over && blockIdx.x == 0 && tid == 0)
        atomicAdd((unsigned long long *)&ctl->fallback_rows, (unsigned long long)total);
    // work items: (tile, range) pairs, ranges of KB_FSPLIT centres when keys are given, else one range of all
    const int nsplit = keys ? (k + KB_FSPLIT - 1) / KB_FSPLIT : 1;
    const int csplit = keys ? KB_FSPLIT : k;
    const uint64_t items = (uint64_t)((total + KB_FR - 1) / KB_FR) * (uint64_t)nsplit;
    for (uint64_t p = blockIdx.x; p < items; p += gridDim.x) {
        const uint32_t t0 = (uint32_t)(p / (uint64_t)nsplit) * KB_FR;
        const int cbeg = (int)(p % (uint64_t)nsplit) * csplit;
        const int cend = (cbeg + csplit < k) ? cbeg + csplit : k;
        const int nr = (int)((total - t0) < (uint32_t)KB_FR ? (total - t0) : (uint32_t)KB_FR);
        __syncthreads();   // the previous tile's rows are no longer read
        if (tid < KB_FR) {
            const uint32_t q = t0 + (tid < nr ? tid : 0);
            rows[tid] = over ? (int64_t)over[q] : (int64_t)q;
        }
        __syncthreads();
        float bst[4];
        uint32_t bl[4];
#pragma unroll
        for (int a = 0; a < 4; a++) {
            bst[a] = INFINITY;
            bl[a] = 0u;
        }
        for (int c0 = cbeg; c0 < cend; c0 += KB_FC) {
            float sacc[4][4];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int b = 0; b < 4; b++) sacc[a][b] = 0.0f;
            for (int j0 = 0; j0 < d; j0 += KB_RCH) {
                const int w = (d - j0) < KB_RCH ? (d - j0) : KB_RCH;
                __syncthreads();
                for (int e = tid; e < KB_FR * KB_RCH; e += 256) {
                    const int r = e / KB_RCH, jj = e - (e / KB_RCH) * KB_RCH;
                    xs[jj][r] = jj < w ? X[rows[r] * d + j0 + jj] : 0.0f;
                }
                for (int e = tid; e < KB_FC * KB_RCH; e += 256) {
                    const int c = e / KB_RCH, jj = e - (e / KB_RCH) * KB_RCH;
                    cs[jj][c] = (jj < w && c0 + c < cend) ? C[(int64_t)(c0 + c) * d + j0 + jj] : 0.0f;
                }
                __syncthreads();
                for (int jj = 0; jj < w; jj++) {
                    float xv[4], cv[4];
#pragma unroll
                    for (int a = 0; a < 4; a++) xv[a] = xs[jj][4 * tr + a];
#pragma unroll
                    for (int b = 0; b < 4; b++) cv[b] = cs[jj][4 * tc + b];
#pragma unroll
                    for (int a = 0; a < 4; a++)
#pragma unroll
                        for (int b = 0; b < 4; b++) {
                            const float t = xv[a] - cv[b];
                            sacc[a][b] = sacc[a][b] + t * t;
                        }
                }
            }
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int c = c0 + 4 * tc + b;
                if (c < cend) {
#pragma unroll
                    for (int a = 0; a < 4; a++)
                        if (sacc[a][b] < bst[a]) {
                            bst[a] = sacc[a][b];
                            bl[a] = (uint32_t)c;
                        }
                }
            }
        }
        // the 16 threads of a row group (consecutive lanes of one wave): smallest value, lowest index on ties
#pragma unroll
        for (int a = 0; a < 4; a++) {
            float v = bst[a];
            uint32_t ix = bl[a];
            for (int off = 8; off > 0; off >>= 1) {
                const float ov = __shfl_xor(v, off);
                const uint32_t oi = (uint32_t)__shfl_xor((int)ix, off);
                if (ov < v || (ov == v && oi < ix)) {
                    v = ov;
                    ix = oi;
                }
            }
            const int r = 4 * tr + a;
            if (tc == 0 && r < nr) {
                if (keys) {
                    if (v < INFINITY)
                        atomicMin((unsigned long long *)&keys[t0 + r],
                                  (unsigned long long)(((uint64_t)__float_as_uint(v) << 32) | ix));
                } else {
                    labels[rows[r]] = ix;
                    best[rows[r]] = v;
                }
            }
        }
    }
}

// The split full scan's keys: (+inf, 0) for every listed row before, its label and best after.
__global__ __launch_bounds__(256) void k_big_fkeys_init(uint64_t *__restrict__ keys, const km_control *__restrict__ ctl,
                                                        const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const uint32_t total = ctl->n_over;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) keys[i] = KB_FKEY0;
}

__global__ __launch_bounds__(256) void k_big_fkeys_fin(const uint64_t *__restrict__ keys,
                                                       const uint32_t *__restrict__ over,
                                                       const km_control *__restrict__ ctl, uint32_t *__restrict__ labels,
                                                       float *__restrict__ best, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const uint32_t total = ctl->n_over;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
        const uint64_t key = keys[i];
        labels[over[i]] = (uint32_t)key;
        best[over[i]] = __uint_as_float((uint32_t)(key >> 32));
    }
}

// ------------------------------------------------------------------ sorted accumulation
//
// A stable counting sort of the rows by label: per 4096-row block a histogram (LDS integer adds, exact), per
// label an exclusive prefix over blocks on top of the labels before it, then each block places its rows in
// ascending row order (rank among earlier rows of the same label in the block). The clusters' float64 sums over
// their rows in that order come from km_chunks.hip (fixed chunks of sorted rows per wave, so an uneven split of
// the rows among the clusters costs nothing). Count, best sum and coordinate sums land as one range sum per entry
// (tmp, S = 1 per slice), the format the finish reads.

static constexpr int KB_RB = 4096;   // rows per histogram / scatter block

// half (may be null): the sort takes only the first 2 *half of the n labels (a count known on the device); blocks
// past them write zero counts.
__device__ __forceinline__ int64_t kb_sort_len(int64_t n, const uint32_t *half) {
    if (!half) return n;
    const int64_t m = 2 * (int64_t)*half;
    return m < n ? m : n;
}

__global__ __launch_bounds__(256) void k_big_hist(const uint32_t *__restrict__ labels, int64_t n, int k,
                                                  uint32_t *__restrict__ H, const uint32_t *__restrict__ half,
                                                  const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    n = kb_sort_len(n, half);
    extern __shared__ uint32_t cnt[];
    for (int c = threadIdx.x; c < k; c += 256) cnt[c] = 0;
    __syncthreads();
    const int64_t r0 = (int64_t)blockIdx.x * KB_RB;
    const int64_t r1 = (r0 + KB_RB < n) ? r0 + KB_RB : n;
    for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) atomicAdd(&cnt[labels[r]], 1u);
    __syncthreads();
    for (int c = threadIdx.x; c < k; c += 256) H[(int64_t)blockIdx.x * k + c] = cnt[c];
}

// The same histogram with the counters in global memory (H zeroed first), for k too large for LDS.
__global__ __launch_bounds__(256) void k_big_hist_g(const uint32_t *__restrict__ labels, int64_t n, int k,
                                                    uint32_t *__restrict__ H, const uint32_t *__restrict__ half,
                                                    const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    n = kb_sort_len(n, half);
    const int64_t r0 = (int64_t)blockIdx.x * KB_RB;
    const int64_t r1 = (r0 + KB_RB < n) ? r0 + KB_RB : n;
    for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) atomicAdd(&H[(int64_t)blockIdx.x * k + labels[r]], 1u);
}

__global__ __launch_bounds__(256) void k_big_zero(uint32_t *__restrict__ p, int64_t n, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) p[e] = 0u;
}

// One block: O[b][c] = (rows with label < c) + (rows with label c in blocks before b); counts[c] = its total.
__global__ __launch_bounds__(1024) void k_big_scan(uint32_t *__restrict__ H, int nb, int k,
                                                   uint32_t *__restrict__ counts, uint32_t *__restrict__ base,
                                                   const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    __shared__ uint32_t part[1024];
    // per label: exclusive prefix over blocks, in place (16 loads in flight before their stores)
    for (int c = threadIdx.x; c < k; c += 1024) {
        uint32_t run = 0;
        for (int b0 = 0; b0 < nb; b0 += 16) {
            uint32_t v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = b0 + u < nb ? H[(int64_t)(b0 + u) * k + c] : 0u;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (b0 + u < nb) {
                    H[(int64_t)(b0 + u) * k + c] = run;
                    run += v[u];
                }
        }
        counts[c] = run;
    }
    __syncthreads();
    // exclusive prefix over labels: each thread a contiguous range, then the range totals in thread order by a
    // scan within each wave and one over the sixteen wave totals (integer sums: any grouping gives the same)
    const int per = (k + 1023) / 1024;
    const int c0 = threadIdx.x * per, c1 = (c0 + per < k) ? c0 + per : k;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t s = 0;
    for (int c = c0; c < c1; c++) s += counts[c];
    uint32_t incl = s;
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63) part[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const uint32_t t = lane < 16 ? part[lane] : 0u;
        uint32_t ti = t;
        for (int off = 1; off < 16; off <<= 1) {
            const uint32_t y = __shfl_up(ti, off);
            if (lane >= off) ti += y;
        }
        if (lane < 16) part[16 + lane] = ti - t;   // the waves before this one
    }
    __syncthreads();
    uint32_t run = part[16 + wave] + incl - s;
    for (int c = c0; c < c1; c++) {
        base[c] = run;
        run += counts[c];
    }
}

// The lanes of this wave holding the same label as this lane (valid lanes only): one ballot per label bit.
__device__ __forceinline__ uint64_t kb_peers(uint32_t L, int nbits, bool valid) {
    uint64_t peers = __ballot(valid);
    for (int b = 0; b < nbits; b++) {
        const bool bit = (L >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
    }
    return peers;
}

// Block per 4096 rows, 256 at a time: a row's place is base[label] + O[b][label] + (rows of its label earlier in
// this block). Within a round of 256, a row's rank among its wave's rows of the same label comes from the peer
// mask; the four waves then take their places in wave order (a barrier between them), the last row of each label
// in a wave advancing that label's running offset.
template <bool GLOBAL_RUN>
__device__ __forceinline__ void kb_scatter_body(const uint32_t *__restrict__ labels, int64_t n, int nbits,
                                                uint32_t *__restrict__ run, const uint32_t *__restrict__ base,
                                                uint32_t *__restrict__ perm) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint64_t lt = (1ull << lane) - 1ull;
    const int64_t r0 = (int64_t)blockIdx.x * KB_RB;
    const int64_t r1 = (r0 + KB_RB < n) ? r0 + KB_RB : n;
    for (int64_t q = r0; q < r1; q += 256) {   // block-uniform trip count: every thread reaches the barriers
        const int64_t r = q + threadIdx.x;
        const bool valid = r < r1;
        const uint32_t L = valid ? labels[r] : 0u;
        const uint64_t peers = kb_peers(L, nbits, valid);
        const uint32_t rank = (uint32_t)__popcll(peers & lt);
        const bool last = (peers & ~lt) == (1ull << lane);   // no peer above this lane
        for (int w = 0; w < 4; w++) {
            __syncthreads();   // the previous wave's offsets are written
            if (wave == w && valid) {
                const uint32_t at = run[L];
                perm[(GLOBAL_RUN ? base[L] : 0u) + at + rank] = (uint32_t)r;
                if (last) run[L] = at + rank + 1;
            }
        }
    }
}

// Running offsets in LDS: run[c] = base[c] + O[b][c].
__global__ __launch_bounds__(256) void k_big_scatter(const uint32_t *__restrict__ labels, int64_t n, int k,
                                                     int nbits, const uint32_t *__restrict__ O,
                                                     const uint32_t *__restrict__ base, uint32_t *__restrict__ perm,
                                                     const uint32_t *__restrict__ half,
                                                     const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    n = kb_sort_len(n, half);
    if ((int64_t)blockIdx.x * KB_RB >= n) return;   // block-uniform: no rows, no barriers
    extern __shared__ uint32_t run[];   // k running offsets
    for (int c = threadIdx.x; c < k; c += 256) run[c] = base[c] + O[(int64_t)blockIdx.x * k + c];
    kb_scatter_body<false>(labels, n, nbits, run, base, perm);
}

// The running offsets in global memory, for k too large for LDS: this block's row of O (O[b][c] + base[c] is the
// next place of label c).
__global__ __launch_bounds__(256) void k_big_scatter_g(const uint32_t *__restrict__ labels, int64_t n, int k,
                                                       int nbits, uint32_t *__restrict__ O,
                                                       const uint32_t *__restrict__ base, uint32_t *__restrict__ perm,
                                                       const uint32_t *__restrict__ half,
                                                       const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    n = kb_sort_len(n, half);
    kb_scatter_body<true>(labels, n, nbits, O + (int64_t)blockIdx.x * k, base, perm);
}

// ------------------------------------------------------------------ planning and launch

typedef void (*screen_fn)(const uint16_t *, const float *, int64_t, int, const uint16_t *, const float *, int, int,
                          int, float, int, const uint32_t *, uint16_t *, uint16_t *, uint32_t *, uint32_t *,
                          km_control *, const int32_t *, float *, int64_t);

template <bool PACK>
static screen_fn kb_screen_for(int DS) {
    switch (DS) {
        case 2: return k_big_screen<2, PACK>;
        case 4: return k_big_screen<4, PACK>;
        case 8: return k_big_screen<8, PACK>;
        case 16: return k_big_screen<16, PACK>;
        case 24: return k_big_screen<24, PACK>;
        case 32: return k_big_screen<32, PACK>;
        case 48: return k_big_screen<48, PACK>;
        case 60: return k_big_screen<60, PACK>;
        case 64: return k_big_screen<64, PACK>;
        case 96: return k_big_screen<96, PACK>;
        default: return nullptr;
    }
}

static int kb_ds(int d) {
    const int s = (d + 15) / 16;
    const int opts[] = {2, 4, 8, 16, 24, 32, 48, 60, 64, 96};   // 60: 960-dim rows without padding to 1024
    for (int o : opts)
        if (s <= o) return o;
    return 0;
}

km_big_plan km_plan_big(int64_t n, int d, int k) {
    km_big_plan pl{};
    if (d <= 16 || d > KM_BIG_MAX_DIMS || k < 1 || k > KM_BIG_MAX_K || n < 1) return pl;
    pl.ok = 1;
    pl.DS = kb_ds(d);
    pl.kpad = (k + 31) / 32 * 32;
    pl.nchunks = pl.kpad / 32;
    int ib = 0;
    while ((1 << ib) < pl.kpad) ib++;
    if (ib < 1) ib = 1;
    pl.ib = k <= KM_BIG_PACK_MAX_K ? ib : 0;
    pl.ntiles = (n + 31) / 32;
    pl.nb = (int)((n + KB_RB - 1) / KB_RB);
    return pl;
}

int km_big_list_slot(int d) { return kb_list_half(kb_ds(d)); }

size_t km_big_x16_elems(const km_big_plan &pl) { return (size_t)pl.ntiles * pl.DS * 64 * 8; }
size_t km_big_cop_elems(const km_big_plan &pl) { return (size_t)pl.nchunks * (pl.DS + 1) * 64 * 8; }

hipError_t km_launch_big_rows(const km_big_plan &pl, const float *X, int64_t n, int d, uint16_t *X16T, float *xsq,
                              hipStream_t s) {
    const int64_t threads = pl.ntiles * pl.DS * 64;
    hipLaunchKernelGGL(k_big_rows, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, X, n, d, pl.DS, X16T,
                       pl.ntiles);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_big_xsq, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, s, X, n, d, xsq);
    return hipGetLastError();
}

hipError_t km_launch_big_xmax(const float *xsq, int64_t n, uint32_t *xmax, hipStream_t s) {
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(k_big_xmax, dim3((unsigned)(blocks < 1024 ? blocks : 1024)), dim3(256), 0, s, xsq, n, xmax);
    return hipGetLastError();
}

hipError_t km_launch_big_centres(const km_big_plan &pl, const float *C, int k, int d, float *csq, float *cn,
                                 uint16_t *Cop, float *maxes, km_control *ctl, const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_big_cnorm, dim3((unsigned)((pl.kpad + 3) / 4)), dim3(256), 0, s, C, k, pl.kpad, d, csq, cn,
                       ctl, stop);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t threads = (int64_t)pl.nchunks * (pl.DS + 1) * 64;
    hipLaunchKernelGGL(k_big_centres, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, C, k, d, pl.DS,
                       pl.nchunks, csq, cn, Cop, maxes, stop);
    return hipGetLastError();
}

hipError_t km_launch_big_screen(const km_big_plan &pl, int mode, const uint16_t *X16T, const float *xsq,
                                const uint32_t *xmax, int64_t n, int d, const uint16_t *Cop, const float *maxes, int k,
                                uint16_t *ncand, uint16_t *cand, uint32_t *over, uint32_t *multi, km_control *ctl,
                                const int32_t *stop, hipStream_t s, float *sraw, int64_t sstride) {
    const bool pack = pl.ib > 0;
    if (sraw && (!pack || sstride < 1)) return hipErrorInvalidValue;
    screen_fn fn = pack ? kb_screen_for<true>(pl.DS) : kb_screen_for<false>(pl.DS);
    if (!fn) return hipErrorInvalidValue;
    const float rho = pack ? (float)(1.01 * (double)(1u << pl.ib) * 0x1p-23) : 0.0f;
    const unsigned blocks = (unsigned)((pl.ntiles + KB_WAVES - 1) / KB_WAVES);
    // exact=False approximates from 64 dims, and only under the half-precision guard (checked in the kernel);
    // below 64 dims the reference's dispatch runs its exact kernels (core.py:2036-2042)
    const int approx = (mode == KM_APPROX && d >= KM_APPROX_MIN_DIMS) ? 1 : 0;
    const int ak = pl.DS + 1, spc = (ak + kb_slice(pl.DS) - 1) / kb_slice(pl.DS), slk = (ak + spc - 1) / spc;
    const size_t lds = 2 * (size_t)slk * 1024 + KB_WAVES * (kb_list_half(pl.DS) + 1) * 64 * (pack ? 4 : 6);
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(64 * KB_WAVES), lds, s, X16T,
                       xsq, n, d, Cop, maxes, k, pl.nchunks, pl.ib, rho, approx, xmax, ncand, cand, over, multi, ctl,
                       stop, sraw, sstride);
    return hipGetLastError();
}

hipError_t km_launch_big_rescore(const float *X, int64_t n, int d, const float *C, int k, const uint16_t *ncand,
                                 const uint16_t *cand, const uint32_t *over, const uint32_t *multi, km_control *ctl,
                                 uint32_t *labels, float *best, int lite, uint64_t *okeys, const int32_t *stop,
                                 hipStream_t s, const km_bnd_refresh *bref) {
    const bool v4 = (d % 4 == 0) && ((uintptr_t)X % 16 == 0) && ((uintptr_t)C % 16 == 0);
    const unsigned chunks = (unsigned)((n + KB_RR - 1) / KB_RR);
    const km_bnd_refresh br = bref ? *bref : km_bnd_refresh{};
    hipError_t e;
    typedef void (*rescore_fn)(const float *, int64_t, int, const float *, int, const uint16_t *, const uint16_t *,
                               int, const uint32_t *, const km_control *, uint32_t *, float *, const int32_t *,
                               km_bnd_refresh);
    const int slot = km_big_list_slot(d);
    if (lite) {
        hipLaunchKernelGGL(k_big_label1, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ncand, cand, n, slot,
                           labels, stop);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        const rescore_fn fn = v4 ? k_big_rescore<true, true> : k_big_rescore<false, true>;
        hipLaunchKernelGGL(fn, dim3(chunks < 16384u ? chunks : 16384u), dim3(KB_RT), 0, s, X, n, d, C, k, ncand, cand,
                           slot, multi, ctl, labels, best, stop, br);
    } else {
        const rescore_fn fn = v4 ? k_big_rescore<true, false> : k_big_rescore<false, false>;
        hipLaunchKernelGGL(fn, dim3(chunks), dim3(KB_RT), 0, s, X, n, d, C, k, ncand, cand, slot,
                           (const uint32_t *)nullptr, ctl, labels, best, stop, br);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (k <= KB_FSPLIT || !okeys) {
        hipLaunchKernelGGL(k_big_fullscan, dim3(1024), dim3(256), 0, s, X, d, C, k, over, (int64_t)0, ctl, labels,
                           best, (uint64_t *)nullptr, stop);
    } else {
        hipLaunchKernelGGL(k_big_fkeys_init, dim3(256), dim3(256), 0, s, okeys, ctl, stop);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(k_big_fullscan, dim3(1024), dim3(256), 0, s, X, d, C, k, over, (int64_t)0, ctl, labels,
                           best, okeys, stop);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(k_big_fkeys_fin, dim3(256), dim3(256), 0, s, okeys, over, ctl, labels, best, stop);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!br.lb) return hipSuccess;
    return km_launch_bnd_overfix(over, ctl, labels, best, br.ub, br.ubl, br.hi, br.bs, stop, s);
}

template <int DS>
static hipError_t kb_launch_screen_bnd(const km_big_plan &pl, const uint16_t *X16T, const float *xsq, int64_t n, int d,
                                       const uint16_t *Cop, const float *maxes, int k, uint16_t *ncand,
                                       uint16_t *cand, uint32_t *over, uint32_t *multi, km_control *ctl,
                                       uint16_t *lb, float *ub, uint32_t *ubl, km_bnd *bs, int cus, hipStream_t s) {
    const float rho = (float)(1.01 * (double)(1u << pl.ib) * 0x1p-23);
    const int ak = DS + 1, spc = (ak + kb_slice(DS) - 1) / kb_slice(DS), slk = (ak + spc - 1) / spc;
    const size_t lds = 2 * (size_t)slk * 1024 + KB_WAVES * (kb_list_half(DS) + 1) * 64 * 4;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)k_big_screen_bnd<DS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds);
        if (e != hipSuccess) return e;
    }
    // one round of blocks on the device (one or two per CU), each looping over its tiles
    const int64_t want = (pl.ntiles + KB_WAVES - 1) / KB_WAVES;
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>(want, (int64_t)cus * (DS > 48 ? 1 : 2)));
    hipLaunchKernelGGL(k_big_screen_bnd<DS>, dim3((unsigned)blocks), dim3(64 * KB_WAVES), lds, s, X16T, xsq, n, d,
                       Cop, maxes, k, pl.nchunks, pl.ib, rho, ncand, cand, over, multi, ctl, lb, ub, ubl,
                       km_bnd_lo(d) * (1.0f - 0x1p-21f), km_bnd_hi(d) * (1.0f + 0x1p-21f), bs);
    return hipGetLastError();
}

hipError_t km_launch_big_screen_bnd(const km_big_plan &pl, const uint16_t *X16T, const float *xsq, int64_t n, int d,
                                    const uint16_t *Cop, const float *maxes, int k, uint16_t *ncand, uint16_t *cand,
                                    uint32_t *over, uint32_t *multi, km_control *ctl, uint16_t *lb, float *ub,
                                    uint32_t *ubl, km_bnd *bs, int cus, hipStream_t s) {
    if (pl.ib <= 0) return hipErrorInvalidValue;   // packed keys only (k <= KM_BIG_PACK_MAX_K)
    switch (pl.DS) {
        case 16: return kb_launch_screen_bnd<16>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 24: return kb_launch_screen_bnd<24>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 32: return kb_launch_screen_bnd<32>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 48: return kb_launch_screen_bnd<48>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 60: return kb_launch_screen_bnd<60>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 64: return kb_launch_screen_bnd<64>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        case 96: return kb_launch_screen_bnd<96>(pl, X16T, xsq, n, d, Cop, maxes, k, ncand, cand, over, multi, ctl, lb, ub, ubl, bs, cus, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t km_launch_rows_tiled(const float *X, int64_t n, int d, const float *C, int k, uint32_t *labels, float *best,
                                const int32_t *stop, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n > (int64_t)0xffffffffu - KB_FR) return hipErrorInvalidValue;
    const int64_t tiles = (n + KB_FR - 1) / KB_FR;
    hipLaunchKernelGGL(k_big_fullscan, dim3((unsigned)(tiles < 2048 ? tiles : 2048)), dim3(256), 0, s, X, d, C, k,
                       (const uint32_t *)nullptr, n, (km_control *)nullptr, labels, best, (uint64_t *)nullptr, stop);
    return hipGetLastError();
}

int64_t km_sorted_blocks(int64_t n) { return (n + KB_RB - 1) / KB_RB; }

hipError_t km_launch_sorted_accum(const float *X, int64_t n, int d, const uint32_t *labels, const float *best, int k,
                                  uint32_t *H, uint32_t *counts, uint32_t *base, uint32_t *perm, double *pieces,
                                  double *tmp, const int32_t *stop, hipStream_t s) {
    if (d < 1 || d > KM_CHUNK_MAX_DIMS) return hipErrorInvalidValue;
    km_big_plan pl{};
    pl.nb = (int)km_sorted_blocks(n);
    return km_launch_big_accum(pl, X, n, d, labels, best, nullptr, k, H, counts, base, perm, pieces, tmp, stop, s);
}

hipError_t km_launch_label_sort(const uint32_t *labels, int64_t n, int k, uint32_t *H, uint32_t *counts,
                                uint32_t *base, uint32_t *perm, const int32_t *stop, hipStream_t s,
                                const uint32_t *half) {
    // counters in LDS up to KM_BIG_PACK_MAX_K labels (16 KB), in global memory above
    const bool glob = k > KM_BIG_PACK_MAX_K;
    const int nb = (int)km_sorted_blocks(n);
    hipError_t e;
    if (glob) {
        const int64_t cells = (int64_t)nb * k;
        hipLaunchKernelGGL(k_big_zero, dim3((unsigned)std::min<int64_t>((cells + 255) / 256, 4096)), dim3(256), 0, s, H,
                           cells, stop);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(k_big_hist_g, dim3(nb), dim3(256), 0, s, labels, n, k, H, half, stop);
    } else {
        hipLaunchKernelGGL(k_big_hist, dim3(nb), dim3(256), (size_t)k * 4, s, labels, n, k, H, half, stop);
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_big_scan, dim3(1), dim3(1024), 0, s, H, nb, k, counts, base, stop);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    int nbits = 1;   // bits of the largest label, k - 1
    while (nbits < 32 && ((uint32_t)(k - 1) >> nbits) != 0u) nbits++;
    if (glob)
        hipLaunchKernelGGL(k_big_scatter_g, dim3(nb), dim3(256), 0, s, labels, n, k, nbits, H, base, perm, half,
                           stop);
    else
        hipLaunchKernelGGL(k_big_scatter, dim3(nb), dim3(256), (size_t)k * 4, s, labels, n, k, nbits, H, base, perm,
                           half, stop);
    return hipGetLastError();
}

hipError_t km_launch_big_accum(const km_big_plan &pl, const float *X, int64_t n, int d, const uint32_t *labels,
                               const float *best, const float *C_lite, int k, uint32_t *H, uint32_t *counts,
                               uint32_t *base, uint32_t *perm, double *pieces, double *tmp, const int32_t *stop,
                               hipStream_t s) {
    if (pl.nb != (int)km_sorted_blocks(n)) return hipErrorInvalidValue;
    hipError_t e = km_launch_label_sort(labels, n, k, H, counts, base, perm, stop, s);
    if (e != hipSuccess) return e;
    return km_launch_chunk_sums(C_lite ? 1 : 0, X, nullptr, 0, d, labels, nullptr, best, C_lite, perm, counts, base, k,
                                nullptr, n, pieces, tmp, stop, s);
}
