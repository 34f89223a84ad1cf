// MFMA-screened exact assignment for gfx950, fused with the per-cluster accumulation.
//
// Per 32-row tile a wave computes a'_c = |c|^2 - 2 x.c for every centre on the matrix cores, in bf16
// (v_mfma_f32_32x32x16_bf16: A = bf16(-2c), 32 centres x 16 dims; B = bf16(x), 16 dims x 32 rows; C = |c|^2).
// That value is only a screen. A rigorous bound on its error, plus the error bound of the float32 direct form,
// gives a window: every centre whose exact float32 direct-form distance could be the row's minimum has a'_c
// inside it. Those candidates - almost always one - are rescored with the direct form in the rows loop's order
// (core.py:263-274), ascending centre index with a strict '<', so labels and best are the rows loop's bit for
// bit. This is the reference's tiles + margin design (core.py:333-377, 675-784) rebuilt for CDNA4: bf16 matrix
// cores instead of fp32 simdgroup MMA, the window derived for that arithmetic, and no n x k matrix in memory.
//
// Lane layout (wave64, one 32-row tile): lane l holds row n = l & 31 of the tile and half h = l >> 5 of its
// dims: [h*DH, h*DH + DH), DH = DP/2. MFMA K-step s (16 contraction slots) takes dims h*DH + 8s + q (q < 8) from
// lane half h; the A operand (centres) is laid out with the same map, so the contraction runs over every dim.
// Accumulator element v (0..15) of tile t in lane l is centre 32t + 8(v/4) + 4h + (v%4) against row n.
//
// Accumulation (ACCUM): the tile's rows go through a per-wave LDS transpose, then rows 2i and 2i+1 are added
// to a per-wave LDS accumulator with one dim per lane (lanes 0-31 row 2i, 32-63 row 2i+1) by Kahan's
// compensated sum; equal labels in a pair are added one after the other. Counts use LDS integer atomics
// (exact, order-free); the inertia is a per-lane Kahan sum. The two waves' accumulators are folded in wave
// order and written as the block's partial. Every accumulator has one writer and a fixed order of adds, so
// the result is the same on every run.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

#define KM_WAVES 2   // waves per block

// ------------------------------------------------------------------ centre preparation

// csq (float32 of the float64 sum), cnorm (|c| rounded up), padding centres get csq = FLT_MAX (never a
// candidate, and finite so packed keys stay ordered numbers), and the bf16(-2c) operand in MFMA A order:
// cb[((t * DS + s) * 64 + lane) * 8 + q] = bf16(-2 * C[32t + (lane & 31), (lane >> 5) * DH + 8s + q]).
__global__ __launch_bounds__(256) void k_prep(const float *__restrict__ C, int k, int d, int kpad, int dpad,
                                              float *__restrict__ csq, float *__restrict__ cnorm,
                                              uint16_t *__restrict__ cb, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int DS = dpad / 16, DH = dpad / 2;
    const int64_t total = (int64_t)kpad * dpad;
    if (e < total) {
        const int q = (int)(e & 7);
        const int lane = (int)((e >> 3) & 63);
        const int64_t ts = e >> 9;
        const int s = (int)(ts % DS), t = (int)(ts / DS);
        const int c = 32 * t + (lane & 31);
        const int j = (lane >> 5) * DH + 8 * s + q;
        float v = 0.0f;
        if (c < k && j < d) v = -2.0f * C[(size_t)c * d + j];
        __bf16 b = (__bf16)v;
        cb[e] = *reinterpret_cast<uint16_t *>(&b);
    }
    if (e < kpad) {
        const int c = (int)e;
        if (c < k) {
            double s = 0.0;
            for (int j = 0; j < d; j++) {
                const double v = C[(size_t)c * d + j];
                s += v * v;
            }
            csq[c] = (float)s;
            cnorm[c] = (float)(sqrt(s) * (1.0 + 1e-6));
        } else {
            csq[c] = 3.0e38f;
            cnorm[c] = 0.0f;
        }
    }
}

// maxes[0] = max |c| (rounded up), maxes[1] = max |c|^2 over the real centres.
__global__ __launch_bounds__(256) void k_prep_max(const float *__restrict__ csq, const float *__restrict__ cnorm,
                                                  int k, float *__restrict__ maxes,
                                                  const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    __shared__ float a[256], b[256];
    float mn = 0.0f, ms = 0.0f;
    for (int c = threadIdx.x; c < k; c += 256) {
        mn = fmaxf(mn, cnorm[c]);
        ms = fmaxf(ms, csq[c]);
    }
    a[threadIdx.x] = mn;
    b[threadIdx.x] = ms;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) {
            a[threadIdx.x] = fmaxf(a[threadIdx.x], a[threadIdx.x + h]);
            b[threadIdx.x] = fmaxf(b[threadIdx.x], b[threadIdx.x + h]);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        maxes[0] = a[0];
        maxes[1] = b[0];
    }
}

hipError_t km_launch_prep(const float *C, int k, int d, int kpad, int dpad, km_centre_aux aux,
                          const int32_t *stop, hipStream_t s) {
    const int64_t total = (int64_t)kpad * dpad;
    const int64_t m = total > kpad ? total : kpad;
    hipLaunchKernelGGL(k_prep, dim3((unsigned)((m + 255) / 256)), dim3(256), 0, s, C, k, d, kpad, dpad, aux.csq,
                       aux.cnorm, aux.cb, stop);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_prep_max, dim3(1), dim3(256), 0, s, aux.csq, aux.cnorm, k, aux.maxes, stop);
    return hipGetLastError();
}

// ------------------------------------------------------------------ the fused kernel

__device__ __forceinline__ float shfl32(float v) { return __shfl_xor(v, 32); }
__device__ __forceinline__ uint32_t shfl32u(uint32_t v) { return (uint32_t)__shfl_xor((int)v, 32); }

// Error-window constants. u = 2^-24 (float32 unit roundoff); gamma_m = m u / (1 - m u).
__host__ __device__ constexpr double km_gamma(int m) { return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08); }

template <int D, int KP, bool ACCUM>
__global__ __launch_bounds__(64 * KM_WAVES) void k_fused_mfma(
    const float *__restrict__ X, int64_t n, const float *__restrict__ C, int k, const float *__restrict__ csq,
    const float *__restrict__ maxes, const uint16_t *__restrict__ cbg, int64_t rbs, uint32_t *__restrict__ labels,
    float *__restrict__ best, float *__restrict__ psum, float *__restrict__ pcomp, int rb0,
    km_control *__restrict__ ctl, const int32_t *__restrict__ stop) {
    constexpr int DP = (D + 15) / 16 * 16;   // padded dims
    constexpr int DH = DP / 2;               // dims per lane half
    constexpr int DS = DP / 16;              // MFMA K-steps
    constexpr int KT = KP / 32;              // centre tiles
    constexpr int NV = KT * 16;              // screen values per lane
    constexpr int IB = NV <= 16 ? 4 : NV <= 32 ? 5 : NV <= 64 ? 6 : 7;   // index bits packed into keys
    constexpr int CS = D + 4;                // LDS row stride of the float32 centres
    constexpr int W = D + 2;
    // window constants (see the derivation in the header of this file and in the design notes)
    constexpr float BETA = (float)(2.0 * (0x1p-8 + 0x1p-18) * (1.0 + 0x1p-20) + 2.01 * km_gamma(DP + 1));
    constexpr float GAM2 = (float)(km_gamma(DP + 1) + 0x1p-24);
    constexpr float GDIR = (float)(km_gamma(D + 2) / (1.0 - km_gamma(D + 2)) * (1.0 + 0x1p-20));
    constexpr float RHO = (float)(1.01 * (double)(1 << IB) * 0x1p-23);
    constexpr float FLUSH = (float)(0x1p-123 * 16.0);   // bf16 denormal flush, times sqrt(DP) <= 16 below
    constexpr float TINY = (float)(DP * 0x1p-118);
    constexpr float XSQ_UP = (float)(1.0 + 2.0 * (DH + 2) * 0x1p-24);
    static_assert(DP <= 64 && KP <= 128, "fused kernel serves dims <= 64 and k <= 128");

    if (stop && *stop) return;

    extern __shared__ float lds[];
    float *Cl = lds;                                       // KP x CS float32 centres
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *wbase = lds + KP * CS + wave * (KP * D * 2 + KP + 32 * D);
    float2 *acc = reinterpret_cast<float2 *>(wbase);       // KP x D (sum, kahan carry)
    uint32_t *cnt = reinterpret_cast<uint32_t *>(wbase + KP * D * 2);   // KP counts
    float *TT = wbase + KP * D * 2 + KP;                   // 32 x D transpose tile

    // centres into LDS (zeros for padding), accumulators cleared
    for (int e = threadIdx.x; e < KP * CS; e += 64 * KM_WAVES) {
        const int c = e / CS, j = e % CS;
        Cl[e] = (c < k && j < D) ? C[(size_t)c * D + j] : 0.0f;
    }
    if (ACCUM) {
        for (int e = lane; e < KP * D; e += 64) acc[e] = make_float2(0.0f, 0.0f);
        for (int e = lane; e < KP; e += 64) cnt[e] = 0u;
    }

    const int rn = lane & 31, h = lane >> 5;
    // resident MFMA operands: A = bf16(-2c) per (tile, k-step); C = |c|^2 of this lane's 16 centres per tile
    bf16x8 Aop[KT][DS];
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int s = 0; s < DS; s++)
            Aop[t][s] = *reinterpret_cast<const bf16x8 *>(cbg + ((size_t)(t * DS + s) * 64 + lane) * 8);
    f32x16 Cin[KT];
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int v = 0; v < 16; v++) Cin[t][v] = csq[32 * t + 8 * (v >> 2) + 4 * h + (v & 3)];
    const float cnmax = maxes[0], csqmax = maxes[1];
    __syncthreads();

    const int64_t r_begin = (int64_t)blockIdx.x * rbs;
    const int64_t r_end = (r_begin + rbs < n) ? r_begin + rbs : n;
    float ine_s = 0.0f, ine_c = 0.0f;   // this lane's Kahan inertia (half 1 lanes)
    uint32_t fallback = 0;              // rows of this lane's tiles rescored against every centre

    for (int64_t r0 = r_begin + (int64_t)wave * 32; r0 < r_end; r0 += 32 * KM_WAVES) {
        const int64_t row = r0 + rn;
        const bool valid = row < r_end;
        // ---- load this lane's half row
        float xf[DH];
        if (D == DP) {   // whole float4s: 16-byte aligned rows (checked by the host)
            const float4 *src = reinterpret_cast<const float4 *>(X + row * D + h * DH);
#pragma unroll
            for (int q = 0; q < DH / 4; q++) {
                const float4 v = valid ? src[q] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                xf[4 * q] = v.x;
                xf[4 * q + 1] = v.y;
                xf[4 * q + 2] = v.z;
                xf[4 * q + 3] = v.w;
            }
        } else {
#pragma unroll
            for (int q = 0; q < DH; q++) {
                const int j = h * DH + q;
                xf[q] = (valid && j < D) ? X[row * D + j] : 0.0f;
            }
        }
        // ---- |x|^2 upper bound and |x| upper bound
        float xs = 0.0f;
#pragma unroll
        for (int q = 0; q < DH; q++) xs = __builtin_fmaf(xf[q], xf[q], xs);
        const float xsq_up = (xs + shfl32(xs)) * XSQ_UP;
        const float nx = __builtin_sqrtf(xsq_up) * (1.0f + 0x1p-22f);
        // ---- screen on the matrix cores
        bf16x8 B[DS];
#pragma unroll
        for (int s = 0; s < DS; s++)
#pragma unroll
            for (int q = 0; q < 8; q++) B[s][q] = (__bf16)xf[8 * s + q];
        f32x16 a[KT];
#pragma unroll
        for (int t = 0; t < KT; t++) {
            a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Aop[t][0], B[0], Cin[t], 0, 0, 0);
#pragma unroll
            for (int s = 1; s < DS; s++) a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Aop[t][s], B[s], a[t], 0, 0, 0);
        }
        // ---- smallest and second smallest screen value, with the local index packed into the low bits
        const uint32_t IMASK = (1u << IB) - 1u;
        float m1 = 3.4e38f, m2 = 3.4e38f;
#pragma unroll
        for (int t = 0; t < KT; t++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float key = __uint_as_float((__float_as_uint(a[t][v]) & ~IMASK) | (uint32_t)(t * 16 + v));
                m2 = __builtin_amdgcn_fmed3f(m1, m2, key);
                m1 = fminf(m1, key);
            }
        const float pm1 = shfl32(m1), pm2 = shfl32(m2);
        const float km = fminf(m1, pm1);
        const float k2 = fminf(fmaxf(m1, pm1), fminf(m2, pm2));
        // index of km: which half holds it, and where
        const uint32_t kmb = __float_as_uint(km) & IMASK;
        const int kh = (m1 == pm1) ? 0 : ((km == m1) ? h : (h ^ 1));   // equal keys: half 0's (either is fine)
        const int kt = (int)kmb >> 4, kv = (int)kmb & 15;
        const int cm = 32 * kt + 8 * (kv >> 2) + 4 * kh + (kv & 3);
        // ---- window
        const float E = BETA * nx * cnmax + GAM2 * csqmax + FLUSH * (nx + cnmax) + TINY;
        const float akm = km + RHO * fabsf(km);
        const float dm_up = fmaxf(0.0f, xsq_up + akm + E) * (1.0f + 0x1p-20f);
        const float margin = (2.0f * E + 2.0f * GDIR * dm_up) * (1.0f + 0x1p-20f) + TINY;
        float T = akm + margin;
        T = T + 0x1p-22f * fabsf(T);
        const bool unique = (k2 - RHO * fabsf(k2)) > T && cm < k;
        // ---- candidate masks (one 32-bit word per centre tile, bit = centre within the tile)
        uint32_t mw[KT];
#pragma unroll
        for (int t = 0; t < KT; t++) mw[t] = (t == kt) ? (1u << (cm & 31)) : 0u;
        const bool any_multi = __ballot(!unique && valid) != 0;
        if (any_multi) {
            uint32_t own_w[KT];
#pragma unroll
            for (int t = 0; t < KT; t++) {
                uint32_t wv = 0;
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float key = __uint_as_float((__float_as_uint(a[t][v]) & ~IMASK) | (uint32_t)(t * 16 + v));
                    if (key - RHO * fabsf(key) <= T) wv |= 1u << (8 * (v >> 2) + 4 * h + (v & 3));
                }
                own_w[t] = wv;
            }
#pragma unroll
            for (int t = 0; t < KT; t++) {
                uint32_t u = own_w[t] | shfl32u(own_w[t]);
                // only real centres
                const int lim = k - 32 * t;
                if (lim < 32) u &= lim <= 0 ? 0u : ((1u << lim) - 1u);
                if (!unique) mw[t] = u;
            }
        }
        bool full = false;
        {
            uint32_t any = 0;
#pragma unroll
            for (int t = 0; t < KT; t++) any |= mw[t];
            full = (any == 0);   // nothing usable (non-finite data): score every centre
        }
        if (full) {
#pragma unroll
            for (int t = 0; t < KT; t++) {
                const int lim = k - 32 * t;
                mw[t] = lim >= 32 ? 0xffffffffu : (lim <= 0 ? 0u : ((1u << lim) - 1u));
            }
        }
        // ---- exact rescoring of the candidates, ascending centre index, strict '<' (the rows loop)
        float bst = INFINITY;
        uint32_t bl = 0;
        uint32_t ncand = 0;
#pragma unroll
        for (int t = 0; t < KT; t++) {
            uint32_t wv = mw[t];
            while (wv) {
                const int b = __builtin_ctz(wv);
                wv &= wv - 1u;
                const int c = 32 * t + b;
                const float *cc = Cl + c * CS;
                float s = 0.0f;
                if (h == 0) {
#pragma unroll
                    for (int q = 0; q < DH; q++) {
                        if (q < D) {
                            const float tq = xf[q] - cc[q];
                            s = s + tq * tq;
                        }
                    }
                }
                const float s0 = shfl32(s);
                if (h == 1) {
                    s = s0;
#pragma unroll
                    for (int q = 0; q < DH; q++) {
                        if (DH + q < D) {
                            const float tq = xf[q] - cc[DH + q];
                            s = s + tq * tq;
                        }
                    }
                    if (s < bst) { bst = s; bl = (uint32_t)c; }
                }
                ncand++;
            }
        }
        // the result lives in half 1; give it to half 0 too
        {
            const float ob = shfl32(bst);
            const uint32_t ol = shfl32u(bl);
            if (h == 0) { bst = ob; bl = ol; }
        }
        if (h == 1 && valid && ncand > 1) fallback++;
        if (valid && h == 1) {
            if (labels) labels[row] = bl;
            if (best) best[row] = bst;
        }
        if (!ACCUM) continue;
        // ---- accumulation
        if (valid && h == 1) {
            atomicAdd(&cnt[bl], 1u);
            const float y = bst - ine_c;
            const float tt = ine_s + y;
            ine_c = (tt - ine_s) - y;
            ine_s = tt;
        }
#pragma unroll
        for (int q = 0; q < DH; q++)
            if (h * DH + q < D) TT[rn * D + h * DH + q] = xf[q];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const uint32_t lab_mine = valid ? bl : 0xffffffffu;
        const int half = lane >> 5, j = lane & 31;
        for (int i = 0; i < 16; i++) {
            const uint32_t L0 = __builtin_amdgcn_readlane(lab_mine, 2 * i);
            const uint32_t L1 = __builtin_amdgcn_readlane(lab_mine, 2 * i + 1);
            if (L0 == 0xffffffffu) break;   // rows past the end come last in a tile
            const uint32_t L = half ? L1 : L0;
            const bool act = (half == 0 || L1 != 0xffffffffu) && j < D;   // D < 32: lanes past D idle
#define KM_KAHAN_UPD()                                              \
    for (int jj = j; jj < D; jj += 32) {                            \
        const float xv = TT[(2 * i + half) * D + jj];               \
        float2 sc = acc[L * D + jj];                                \
        const float y = xv - sc.y;                                  \
        const float tt = sc.x + y;                                  \
        sc.y = (tt - sc.x) - y;                                     \
        sc.x = tt;                                                  \
        acc[L * D + jj] = sc;                                       \
    }
            if (L0 != L1) {
                if (act) KM_KAHAN_UPD();
            } else {
                if (act && half == 0) KM_KAHAN_UPD();
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                if (act && half == 1) KM_KAHAN_UPD();
            }
#undef KM_KAHAN_UPD
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    }

    if (fallback) atomicAdd((unsigned long long *)&ctl->fallback_rows, (unsigned long long)fallback);
    if (!ACCUM) return;

    // ---- fold the waves' accumulators in wave order and write this block's partial
    // inertia: fixed-order reduction of the lanes' (s, c), then waves in order
    __shared__ float ine_w[KM_WAVES * 2];
    {
        float s = (h == 1) ? ine_s : 0.0f;
        float c = (h == 1) ? -ine_c : 0.0f;   // Kahan carry c means the true sum is s - c
        for (int off = 32; off > 0; off >>= 1) {
            const float so = __shfl_xor(s, off), co = __shfl_xor(c, off);
            // combine in lane order: lower half first
            const float a0 = (lane & off) ? so : s, a1 = (lane & off) ? s : so;
            const float c0 = (lane & off) ? co : c, c1 = (lane & off) ? c : co;
            const float tt = a0 + a1;
            const float err = (fabsf(a0) >= fabsf(a1)) ? ((a0 - tt) + a1) : ((a1 - tt) + a0);
            s = tt;
            c = c0 + c1 + err;
        }
        if (lane == 0) {
            ine_w[wave * 2] = s;
            ine_w[wave * 2 + 1] = c;
        }
    }
    __syncthreads();
    const int64_t kw = (int64_t)k * W;
    float *ps = psum + (int64_t)(rb0 + blockIdx.x) * kw;
    float *pc = pcomp + (int64_t)(rb0 + blockIdx.x) * kw;
    for (int e = threadIdx.x; e < k * W; e += 64 * KM_WAVES) {
        const int c = e / W, col = e % W;
        float s = 0.0f, cc = 0.0f;
        if (col == 0) {
            uint32_t tot = 0;
            for (int w = 0; w < KM_WAVES; w++)
                tot += reinterpret_cast<const uint32_t *>(lds + KP * CS + w * (KP * D * 2 + KP + 32 * D) + KP * D * 2)[c];
            s = (float)tot;
        } else if (col == 1) {
            if (c == 0) {
                for (int w = 0; w < KM_WAVES; w++) {
                    const float v = ine_w[2 * w], vc = ine_w[2 * w + 1];
                    const float tt = s + v;
                    cc += (fabsf(s) >= fabsf(v)) ? ((s - tt) + v) : ((v - tt) + s);
                    cc += vc;
                    s = tt;
                }
            }
        } else {
            const int jj = col - 2;
            for (int w = 0; w < KM_WAVES; w++) {
                const float2 sc = reinterpret_cast<const float2 *>(lds + KP * CS + w * (KP * D * 2 + KP + 32 * D))[c * D + jj];
                const float v = sc.x, vc = -sc.y;   // Kahan: true = x - carry
                const float tt = s + v;
                cc += (fabsf(s) >= fabsf(v)) ? ((s - tt) + v) : ((v - tt) + s);
                cc += vc;
                s = tt;
            }
        }
        ps[e] = s;
        pc[e] = cc;
    }
}

// ------------------------------------------------------------------ planning and launch

template <int D, int KP, bool ACCUM>
static size_t fused_lds() {
    constexpr int CS = D + 4;
    return (size_t)(KP * CS + KM_WAVES * (KP * D * 2 + KP + 32 * D)) * sizeof(float);
}

typedef void (*fused_fn)(const float *, int64_t, const float *, int, const float *, const float *, const uint16_t *,
                         int64_t, uint32_t *, float *, float *, float *, int, km_control *, const int32_t *);

struct fused_entry {
    int d, kp;
    fused_fn acc, noacc;
    size_t lds;
};

#define KM_FUSED(DD, KK) \
    {DD, KK, k_fused_mfma<DD, KK, true>, k_fused_mfma<DD, KK, false>, 0}

static fused_entry g_fused[] = {
    KM_FUSED(16, 32), KM_FUSED(16, 64), KM_FUSED(16, 128),
    KM_FUSED(32, 32), KM_FUSED(32, 64),
    KM_FUSED(64, 32),
};
#undef KM_FUSED

static size_t lds_for(int d, int kp) {
    return (size_t)(kp * (d + 4) + KM_WAVES * (kp * d * 2 + kp + 32 * d)) * sizeof(float);
}

static const fused_entry *find_fused(int d, int k) {
    const int kp = (k + 31) / 32 * 32;
    for (auto &e : g_fused)
        if (e.d == d && e.kp >= kp && (e.kp == kp || (kp <= 32 ? e.kp == 32 : kp <= 64 ? e.kp == 64 : e.kp == 128)))
            return &e;
    return nullptr;
}

static int g_cus = 0;
static size_t g_lds_max = 0;

km_mfma_plan km_plan_mfma(int64_t n, int d, int k, int fused) {
    (void)fused;
    km_mfma_plan pl{};
    const fused_entry *fe = find_fused(d, k);
    if (!fe || n < 1) return pl;
    pl.ok = 1;
    pl.kpad = fe->kp;
    pl.dpad = (d + 15) / 16 * 16;
    pl.lds = lds_for(d, fe->kp);
    if (g_cus == 0) {
        int dev = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
            g_cus = prop.multiProcessorCount;
        if (g_cus <= 0) g_cus = 256;
        g_lds_max = (size_t)prop.sharedMemPerBlock;
        if (g_lds_max == 0) g_lds_max = 65536;
    }
    if (pl.lds > g_lds_max) {
        pl.ok = 0;
        return pl;
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)fe->acc, 64 * KM_WAVES, pl.lds) != hipSuccess ||
        occ < 1)
        occ = 1;
    const int64_t slots = (int64_t)g_cus * occ;
    const int64_t tiles = (n + 63) / 64;   // 64-row units (one per wave pair step)
    int64_t nrb = tiles < slots ? tiles : slots;
    if (nrb < 1) nrb = 1;
    int64_t rbs = (n + nrb - 1) / nrb;
    rbs = (rbs + 63) / 64 * 64;
    pl.rbs = rbs;
    pl.nrb = (int)((n + rbs - 1) / rbs);
    return pl;
}

hipError_t km_launch_mfma(const km_mfma_plan &pl, int fused, const float *X, int64_t n, int d, const float *C, int k,
                          km_centre_aux aux, uint32_t *labels, float *best, float *psum, float *pcomp, int rb0,
                          km_control *ctl, const int32_t *stop, hipStream_t s) {
    const fused_entry *fe = find_fused(d, k);
    if (!fe || !pl.ok) return hipErrorInvalidValue;
    fused_fn fn = fused ? fe->acc : fe->noacc;
    hipLaunchKernelGGL(fn, dim3(pl.nrb), dim3(64 * KM_WAVES), pl.lds, s, X, n, C, k, aux.csq, aux.maxes, aux.cb, pl.rbs,
                       labels, best, psum, pcomp, rb0, ctl, stop);
    return hipGetLastError();
}
