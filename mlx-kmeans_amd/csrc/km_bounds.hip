// Per-centre lower bounds between Lloyd passes for the exact wide-row path: the reference's Elkan bounds
// (core.py:1690-2015, gated at 2063-2084) rebuilt around this engine's screen and exact rescoring.
//
// State (per data set and k, kept by the context):
//   lb[row][c]  float16 lower bound, rounded toward zero, in a frame: lb - S_c <= sqrt(D_c) (1 - g), with D_c the
//               exact squared distance of the row to centre c now, g the rows loop's relative error (gamma_{d+2})
//               and S_c the centre's drift summed since the frame began (each pass's |c' - c|, rounded up; the
//               triangle inequality moves sqrt(D_c) by at most that much)
//   ub[row], ubl[row]   ub >= sqrt(D_l) (1 + g) for the centre l = ubl (raised by l's drift each pass)
// The frame begins at every screened pass (S = 0), whose screen writes lb from its matrix-core values and their
// error bound E (D_c >= |x|^2 + a'_c - E) and ub from the screen minimiser's upper bound.
//
// A pass on the bounds lists, per row, every centre c with lb_c - S_c not above ub. Every other centre has
// sqrt(D_c) (1 - g) > sqrt(D_l) (1 + g), so its direct-form distance s_c >= D_c (1 - g) exceeds s_l <= D_l (1 + g)
// strictly: it can neither be the rows loop's minimum nor tie it (and l itself is listed, lb_l <= ub). The rows
// loop restricted to the listed centres (k_big_rescore, ascending index, strict '<') therefore returns the rows
// loop's label and distance bit for bit; a row with one listed centre has that label. The exact distances the
// rescoring computes refresh the listed bounds (and ub), as the reference's step kernel rewrites them
// (core.py:1828-1853). Unlike the reference, whose step keeps the old label unless a visited centre is strictly
// nearer, the result here is the rows loop's on ties too.
//
// When (the reference's policy, core.py:2063-2106): every screened pass writes the bounds of a strided sample of
// 32-row tiles (KM_BND_SAMPLE_TILES of them, the reference's 8192 sampled rows) and every row's ub. The next pass
// first counts, on the sample, the pairs its bounds would visit. If every tile has bounds and at most
// max_visited (BOUNDS_MAX_VISITED = 5 %, core.py:516) of the pairs would be visited, the pass runs on the bounds;
// if the sample says bounds built now would pay, the pass screens and writes every tile's bounds (the reference's
// build, core.py:2091-2096); bounds whose sample has decayed past the threshold are dropped (core.py:2075-2079).
#pragma clang fp contract(off)
#include "km_internal.h"
#include "kmeans_hip.h"
#include <math.h>

#include <algorithm>

namespace {

constexpr int KD_HALF = 16;              // candidates per half-row (the screen's KB_HALF)
constexpr int KD_CAP = 2 * KD_HALF;      // per row
constexpr int KD_OVER = 0xffff;          // ncand: scan every centre

typedef _Float16 kd_h8 __attribute__((ext_vector_type(8)));

__host__ __device__ constexpr double kd_gamma(int m) {
    return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08);
}

// The raised upper bound of a row: ub + hi * drift of its centre, rounded up; +inf when not finite.
__device__ __forceinline__ float kd_raise(float u, float dl, float hi) {
    const float r = (u + dl * hi) * (1.0f + 0x1p-22f);
    return r < INFINITY ? r : INFINITY;
}

// Wave per 32-row tile, lane per half-row (row 32 t + lane % 32, centres of half lane / 32 of each chunk, the
// screen's order). Every listed centre c: lb_c - S_c not above ub (a NaN difference lists the centre). COUNT: the
// listed pairs (the ub centre excluded, a row with no finite ub counting every centre) into bs; else the candidate
// lists and each row's raised ub.
template <bool COUNT>
__global__ __launch_bounds__(256) void k_bnd_scan(const uint16_t *__restrict__ lb, float *__restrict__ ub,
                                                  const uint32_t *__restrict__ ubl, int64_t n, int k, int nchunks,
                                                  int64_t tstride, const float *__restrict__ S,
                                                  const float *__restrict__ delta, float hi,
                                                  uint16_t *__restrict__ ncand, uint16_t *__restrict__ cand,
                                                  uint32_t *__restrict__ over, uint32_t *__restrict__ multi,
                                                  km_control *__restrict__ ctl, km_bnd *__restrict__ bs,
                                                  const int32_t *__restrict__ gate) {
    if (gate && *gate) return;
    extern __shared__ float Sp[];   // S in the screen's order: Sp[32 ch + 16 h + v] = S[km_bnd_centre(ch, h, v)]
    const int kpad = 32 * nchunks;
    for (int p = threadIdx.x; p < kpad; p += 256) {
        const int c = km_bnd_centre(p >> 5, (p >> 4) & 1, p & 15);
        Sp[p] = c < k ? S[c] : -INFINITY;   // padding centres: never listed
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int64_t ntiles = (n + 31) / 32;
    const int64_t nwork = (ntiles + tstride - 1) / tstride;
    unsigned long long vis = 0, prs = 0;
    for (int64_t w = (int64_t)blockIdx.x * 4 + wave; w < nwork; w += (int64_t)gridDim.x * 4) {
        const int64_t tile = w * tstride;
        const int64_t row = tile * 32 + (lane & 31);
        const bool real = row < n;
        float u = INFINITY;
        if (real) {
            const uint32_t l = ubl[row];
            u = kd_raise(ub[row], l < (uint32_t)k ? delta[l] : INFINITY, hi);
        }
        const bool fin = u < INFINITY;
        const kd_h8 *lp = reinterpret_cast<const kd_h8 *>(lb + ((tile * nchunks) * 64 + lane) * 16);
        int cnt = 0;
        uint32_t nv = 0;
        uint16_t *mine = cand + row * KD_CAP + h * KD_HALF;
        for (int ch = 0; ch < nchunks; ch++) {
            const kd_h8 a = __builtin_nontemporal_load(lp + ch * 128);
            const kd_h8 b = __builtin_nontemporal_load(lp + ch * 128 + 1);
            const float *sp = Sp + 32 * ch + 16 * h;
            uint32_t mask = 0;
#pragma unroll
            for (int v = 0; v < 8; v++) {
                mask |= (!(((float)a[v] - sp[v]) > u)) ? (1u << v) : 0u;
                mask |= (!(((float)b[v] - sp[v + 8]) > u)) ? (1u << (v + 8)) : 0u;
            }
            if (!real || !fin) mask = 0;
            if (COUNT) {
                nv += (uint32_t)__popc(mask);
            } else {
                while (mask) {
                    const int v = __ffs(mask) - 1;
                    mask &= mask - 1u;
                    if (cnt < KD_HALF) mine[cnt] = (uint16_t)km_bnd_centre(ch, h, v);
                    cnt++;
                }
            }
        }
        if (COUNT) {
            const uint32_t tot = nv + (uint32_t)__shfl_xor((int)nv, 32);
            if (h == 0 && real) {
                vis += fin ? (tot > 0 ? tot - 1u : 0u) : (unsigned long long)k;
                prs += (unsigned long long)k;
            }
            continue;
        }
        const int cnt_o = __shfl_xor(cnt, 32);
        if (!real || h != 0) continue;
        int code;
        if (!fin || cnt > KD_HALF || cnt_o > KD_HALF || cnt + cnt_o == 0) code = KD_OVER;
        else code = cnt | (cnt_o << 8);
        ub[row] = u;
        ncand[row] = (uint16_t)code;
        if (code == KD_OVER) over[atomicAdd(&ctl->n_over, 1u)] = (uint32_t)row;
        if (code != KD_OVER && cnt + cnt_o >= 2) multi[atomicAdd(&ctl->n_multi, 1u)] = (uint32_t)row;
    }
    if (COUNT) {
        for (int off = 32; off > 0; off >>= 1) {
            vis += __shfl_xor(vis, off);
            prs += __shfl_xor(prs, off);
        }
        if (lane == 0 && prs) {
            atomicAdd(&bs->visits, vis);
            atomicAdd(&bs->pairs, prs);
        }
    }
}

// Wave per centre: delta_c = |C_c - Clast_c| (float64 sum over dims, rounded up; +inf when not finite), S_c += delta_c
// (rounded up), Clast_c = C_c. valid == 0: a new state (S = 0, nothing sampled or built).
__global__ __launch_bounds__(256) void k_bnd_drift(const float *__restrict__ C, float *__restrict__ Clast, int k, int d,
                                                   int valid, float *__restrict__ S, float *__restrict__ delta,
                                                   km_bnd *__restrict__ bs, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        bs->visits = 0;
        bs->pairs = 0;
        if (!valid) {
            bs->sample_ok = 0;
            bs->built = 0;
        }
    }
    const int c = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (c >= k) return;
    const float *cr = C + (int64_t)c * d;
    float *lr = Clast + (int64_t)c * d;
    double s = 0.0;
    for (int j = lane; j < d; j += 64) {
        const double t = (double)cr[j] - (double)lr[j];
        s += t * t;
        lr[j] = cr[j];   // this lane's own dims: read before written
    }
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) {
        float dl = (float)(sqrt(s) * (1.0 + 0x1p-20));
        if (!(dl < INFINITY)) dl = INFINITY;
        delta[c] = valid ? dl : 0.0f;
        const float sn = (S[c] + dl) * (1.0f + 0x1p-21f);
        S[c] = valid ? (sn < INFINITY ? sn : INFINITY) : 0.0f;
    }
}

// One block: this pass's mode from the sample (see the file's head), the gates, the counters; a screened pass
// begins a new frame (S = 0). When the loop has stopped every gate closes.
__global__ __launch_bounds__(256) void k_bnd_decide(km_bnd *__restrict__ bs, double max_visited, float *__restrict__ S,
                                                    int k, const int32_t *__restrict__ stop) {
    __shared__ int s_screen;
    if (stop && *stop) {
        if (threadIdx.x == 0) {
            bs->skip_plain = 1;
            bs->skip_bscreen = 1;
            bs->skip_list = 1;
        }
        return;
    }
    if (threadIdx.x == 0) {
        const double f = (bs->sample_ok && bs->pairs) ? (double)bs->visits / (double)bs->pairs : 1.0;
        bs->last_frac = f;
        bs->n_tracked++;
        const bool pays = f <= max_visited;
        if (bs->built && pays) {   // a pass on the bounds
            bs->skip_plain = 1;
            bs->skip_bscreen = 1;
            bs->skip_list = 0;
            bs->build = 0;
            bs->n_bounds++;
            s_screen = 0;
        } else {                   // a screened pass: build when the sample says bounds built now would pay
            const int build = (!bs->built && bs->sample_ok && pays) ? 1 : 0;
            bs->build = build;
            bs->built = build;
            bs->n_builds += build;
            bs->skip_plain = build;
            bs->skip_bscreen = 0;
            bs->skip_list = 1;
            bs->sample_ok = 1;     // this pass's screen writes the sample tiles
            s_screen = 1;
        }
    }
    __syncthreads();
    if (s_screen)
        for (int c = threadIdx.x; c < k; c += 256) S[c] = 0.0f;
}

// After the full scan: the overflow rows' ub from their exact distance (the rows loop's best), when the bounds
// describe every tile.
__global__ __launch_bounds__(256) void k_bnd_overfix(const uint32_t *__restrict__ over,
                                                     const km_control *__restrict__ ctl,
                                                     const uint32_t *__restrict__ labels, const float *__restrict__ best,
                                                     float *__restrict__ ub, uint32_t *__restrict__ ubl, float hi,
                                                     const km_bnd *__restrict__ bs, const int32_t *__restrict__ stop) {
    if ((stop && *stop) || !bs->built) return;
    const uint32_t total = ctl->n_over;
    for (uint32_t i = blockIdx.x * 256 + threadIdx.x; i < total; i += gridDim.x * 256) {
        const uint32_t r = over[i];
        const float b = best[r];
        const float u = (b >= 0.0f && b < INFINITY) ? __builtin_sqrtf(b) * hi : INFINITY;
        ub[r] = u < INFINITY ? u : INFINITY;
        ubl[r] = labels[r];
    }
}

}  // namespace

// lo <= (1 - g) (1 - 2^-20): with g = gamma_{d+2}, the rows loop's relative error, and room for the square root's
// rounding and the float32 products that form a bound; hi >= (1 + g) (1 + 2^-20) likewise
float km_bnd_lo(int d) { return (float)(1.0 - 2.0 * kd_gamma(d + 2) - 0x1p-19); }
float km_bnd_hi(int d) { return (float)(1.0 + 2.0 * kd_gamma(d + 2) + 0x1p-19); }

hipError_t km_launch_bnd_drift(const float *C, float *Clast, int k, int d, int valid, float *S, float *delta,
                               km_bnd *bs, const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_drift, dim3((unsigned)((k + 3) / 4)), dim3(256), 0, s, C, Clast, k, d, valid, S, delta, bs,
                       stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_count(const uint16_t *lb, const float *ub, const uint32_t *ubl, int64_t n, int k,
                               int nchunks, int64_t tstride, const float *S, const float *delta, float hi,
                               km_bnd *bs, const int32_t *stop, int cus, hipStream_t s) {
    const int64_t nwork = ((n + 31) / 32 + tstride - 1) / tstride;
    const int64_t blocks = std::min<int64_t>((nwork + 3) / 4, (int64_t)cus * 4);
    hipLaunchKernelGGL(k_bnd_scan<true>, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256),
                       (size_t)nchunks * 32 * sizeof(float), s, lb, const_cast<float *>(ub), ubl, n, k, nchunks,
                       tstride, S, delta, hi, (uint16_t *)nullptr, (uint16_t *)nullptr, (uint32_t *)nullptr,
                       (uint32_t *)nullptr, (km_control *)nullptr, bs, stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_decide(km_bnd *bs, double max_visited, float *S, int k, const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_decide, dim3(1), dim3(256), 0, s, bs, max_visited, S, k, stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_list(const uint16_t *lb, float *ub, const uint32_t *ubl, int64_t n, int k, int nchunks,
                              const float *S, const float *delta, float hi, uint16_t *ncand, uint16_t *cand,
                              uint32_t *over, uint32_t *multi, km_control *ctl, km_bnd *bs, int cus, hipStream_t s) {
    const int64_t nwork = (n + 31) / 32;
    const int64_t blocks = std::min<int64_t>((nwork + 3) / 4, (int64_t)cus * 16);
    hipLaunchKernelGGL(k_bnd_scan<false>, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256),
                       (size_t)nchunks * 32 * sizeof(float), s, lb, ub, ubl, n, k, nchunks, (int64_t)1, S, delta, hi,
                       ncand, cand, over, multi, ctl, bs, &bs->skip_list);
    return hipGetLastError();
}

hipError_t km_launch_bnd_overfix(const uint32_t *over, const km_control *ctl, const uint32_t *labels,
                                 const float *best, float *ub, uint32_t *ubl, float hi, const km_bnd *bs,
                                 const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_overfix, dim3(64), dim3(256), 0, s, over, ctl, labels, best, ub, ubl, hi, bs, stop);
    return hipGetLastError();
}
