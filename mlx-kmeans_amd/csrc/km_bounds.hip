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
// When (the reference's policy, core.py:2063-2106): a strided sample of 32-row tiles (KM_BND_SAMPLE_TILES of them,
// 2048 rows where the reference samples 8192) has bounds at every tracked pass: each pass first counts, on the
// sample, the pairs the bounds kept from the earlier passes would visit now (k_bnd_count); a screened pass then
// rewrites the sample's bounds from the raw screen values the plain screen stored for those tiles (k_bnd_resample),
// a build from its own, a pass on the bounds refreshes them as every row's. If every tile has bounds and at most
// max_visited (BOUNDS_MAX_VISITED = 5 %, core.py:516)
// of the pairs would be visited, the pass runs on the bounds; if the sample says bounds built at the previous pass
// would pay, the pass screens and writes every tile's bounds (the reference's build, core.py:2091-2096, in a new
// frame: S = 0); bounds whose sample has decayed past the threshold are dropped (core.py:2075-2079).
#pragma clang fp contract(off)
#include "km_internal.h"
#include "kmeans_hip.h"
#include <math.h>

#include <algorithm>

namespace {

constexpr int KD_OVER = 0xffff;          // ncand: scan every centre

typedef _Float16 kd_h8 __attribute__((ext_vector_type(8)));


// The raised upper bound of a row: ub + hi * drift of its centre, rounded up; +inf when not finite.
__device__ __forceinline__ float kd_raise(float u, float dl, float hi) {
    const float r = (u + dl * hi) * (1.0f + 0x1p-22f);
    return r < INFINITY ? r : INFINITY;
}

// Wave per 32-row tile, lane per half-row (row 32 t + lane % 32, centres of half lane / 32 of each chunk, the
// screen's order): every centre c with lb_c - S_c not above ub goes to the row's candidate lists (as the screen
// writes them: at most `slot` per half-row, else the row takes the full scan, as does a row without a finite ub),
// and the raised ub is written back.
__global__ __launch_bounds__(256) void k_bnd_list(const uint16_t *__restrict__ lb, float *__restrict__ ub,
                                                  const uint32_t *__restrict__ ubl, int64_t n, int k, int nchunks,
                                                  const float *__restrict__ S, const float *__restrict__ delta,
                                                  float hi, uint16_t *__restrict__ ncand, uint16_t *__restrict__ cand,
                                                  int slot, uint32_t *__restrict__ over, uint32_t *__restrict__ multi,
                                                  km_control *__restrict__ ctl, const int32_t *__restrict__ gate) {
    if (*gate) return;
    extern __shared__ float Sp[];   // S in the screen's order: Sp[32 ch + 16 h + v] = S[km_bnd_centre(ch, h, v)]
    const int kpad = 32 * nchunks;
    for (int p = threadIdx.x; p < kpad; p += 256) {
        const int c = km_bnd_centre(p >> 5, (p >> 4) & 1, p & 15);
        Sp[p] = c < k ? S[c] : -INFINITY;   // padding centres: never listed
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int64_t ntiles = (n + 31) / 32;
    for (int64_t tile = (int64_t)blockIdx.x * 4 + wave; tile < ntiles; tile += (int64_t)gridDim.x * 4) {
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
        uint16_t *mine = cand + row * (2 * slot) + h * slot;
        // Two chunks per step (four 16-byte loads in flight per lane). Per chunk the smallest lb - S first (lb is
        // finite or -inf and S not NaN; a NaN difference, padding against padding, is never listed); only a chunk
        // with one at or below ub is looked at value by value.
        auto chunk = [&](int ch, const kd_h8 &a, const kd_h8 &b) {
            const float *sp = Sp + 32 * ch + 16 * h;
            float t[16];
#pragma unroll
            for (int v = 0; v < 8; v++) {
                t[v] = (float)a[v] - sp[v];
                t[v + 8] = (float)b[v] - sp[v + 8];
            }
            float mn = t[0];
#pragma unroll
            for (int v = 1; v < 16; v++) mn = fminf(mn, t[v]);
            if (mn > u || !real || !fin) return;
            uint32_t mask = 0;
#pragma unroll
            for (int v = 0; v < 16; v++) mask |= (t[v] <= u) ? (1u << v) : 0u;
            while (mask) {
                const int v = __ffs(mask) - 1;
                mask &= mask - 1u;
                if (cnt < slot) mine[cnt] = (uint16_t)km_bnd_centre(ch, h, v);
                cnt++;
            }
        };
        int ch = 0;
        for (; ch + 1 < nchunks; ch += 2) {
            const kd_h8 a0 = __builtin_nontemporal_load(lp + ch * 128);
            const kd_h8 b0 = __builtin_nontemporal_load(lp + ch * 128 + 1);
            const kd_h8 a1 = __builtin_nontemporal_load(lp + ch * 128 + 128);
            const kd_h8 b1 = __builtin_nontemporal_load(lp + ch * 128 + 129);
            chunk(ch, a0, b0);
            chunk(ch + 1, a1, b1);
        }
        if (ch < nchunks) {
            const kd_h8 a0 = __builtin_nontemporal_load(lp + ch * 128);
            const kd_h8 b0 = __builtin_nontemporal_load(lp + ch * 128 + 1);
            chunk(ch, a0, b0);
        }
        const int cnt_o = __shfl_xor(cnt, 32);
        const bool mine_row = real && h == 0;
        int code = KD_OVER;
        if (mine_row) {
            if (fin && cnt <= slot && cnt_o <= slot && cnt + cnt_o > 0) code = cnt | (cnt_o << 8);
            ub[row] = u;
            ncand[row] = (uint16_t)code;
        }
        // the full-scan and several-candidate lists: one counter update per wave and list
        const bool is_over = mine_row && code == KD_OVER;
        const bool is_multi = mine_row && code != KD_OVER && cnt + cnt_o >= 2;
        const uint64_t mo = __ballot(is_over), mm = __ballot(is_multi);
        const uint64_t below = (1ull << lane) - 1ull;
        if (mo) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&ctl->n_over, (uint32_t)__popcll(mo));
            base = (uint32_t)__shfl((int)base, 0);
            if (is_over) over[base + (uint32_t)__popcll(mo & below)] = (uint32_t)row;
        }
        if (mm) {
            uint32_t base = 0;
            if (lane == 0) base = atomicAdd(&ctl->n_multi, (uint32_t)__popcll(mm));
            base = (uint32_t)__shfl((int)base, 0);
            if (is_multi) multi[base + (uint32_t)__popcll(mm & below)] = (uint32_t)row;
        }
    }
}

// The sample kernels take a block of KD_SW waves per sample tile (t = b tstride): wave w the chunks w, w + KD_SW, ...,
// lane the half-row (row 32 t + lane % 32, half lane / 32, the screen's order), the per-row results met in LDS.
constexpr int KD_SW = 16;

// The (row, centre) pairs the stored bounds would visit now (lb_c - S_c not above the raised ub), the ub centre
// excluded, a row without a finite ub counting every centre.
__global__ __launch_bounds__(64 * KD_SW) void k_bnd_count(const uint16_t *__restrict__ lb, const float *__restrict__ ub,
                                                          const uint32_t *__restrict__ ubl, int64_t n, int k,
                                                          int nchunks, int64_t tstride, const float *__restrict__ S,
                                                          const float *__restrict__ delta, float hi,
                                                          km_bnd *__restrict__ bs, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    extern __shared__ float Sp[];
    __shared__ uint32_t s_cnt[KD_SW][64];
    const int kpad = 32 * nchunks;
    for (int p = threadIdx.x; p < kpad; p += 64 * KD_SW) {
        const int c = km_bnd_centre(p >> 5, (p >> 4) & 1, p & 15);
        Sp[p] = c < k ? S[c] : -INFINITY;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int64_t tile = (int64_t)blockIdx.x * tstride;
    const int64_t row = tile * 32 + (lane & 31);
    const bool real = row < n;
    float u = INFINITY;
    if (real) {
        const uint32_t l = ubl[row];
        u = kd_raise(ub[row], l < (uint32_t)k ? delta[l] : INFINITY, hi);
    }
    const kd_h8 *lp = reinterpret_cast<const kd_h8 *>(lb + ((tile * nchunks) * 64 + lane) * 16);
    uint32_t nv = 0;
    for (int ch = wave; ch < nchunks; ch += KD_SW) {
        const kd_h8 a = lp[ch * 128], b = lp[ch * 128 + 1];
        const float *sp = Sp + 32 * ch + 16 * h;
#pragma unroll
        for (int v = 0; v < 8; v++) {
            nv += ((float)a[v] - sp[v] <= u) ? 1u : 0u;
            nv += ((float)b[v] - sp[v + 8] <= u) ? 1u : 0u;
        }
    }
    s_cnt[wave][lane] = nv;
    __syncthreads();
    if (wave != 0) return;
    unsigned long long vis = 0, prs = 0;
    if (real && h == 0) {
        uint32_t tot = 0;
        for (int w = 0; w < KD_SW; w++) tot += s_cnt[w][lane] + s_cnt[w][lane + 32];
        vis = u < INFINITY ? (tot > 0 ? tot - 1u : 0u) : (unsigned long long)k;
        prs = (unsigned long long)k;
    }
    for (int off = 32; off > 0; off >>= 1) {
        vis += __shfl_xor(vis, off);
        prs += __shfl_xor(prs, off);
    }
    if (lane == 0 && prs) {
        atomicAdd(&bs->visits, vis);
        atomicAdd(&bs->pairs, prs);
    }
}

// After a plain screen that stored the sample tile's raw values a'_c: the bounds sqrt(|x|^2 + a'_c - E) lo + S_c (the
// current frame; rounded toward zero; 0 for a centre whose drift is not finite, the largest for padding centres) and
// ub / ubl from the smallest a'_c, as the building screen writes them.
__global__ __launch_bounds__(64 * KD_SW) void k_bnd_resample(const float *__restrict__ sraw,
                                                             const float *__restrict__ xsq, int64_t n, km_screen_k q,
                                                             const float *__restrict__ maxes, int k, int nchunks,
                                                             int64_t tstride, uint16_t *__restrict__ lb,
                                                             float *__restrict__ ub, uint32_t *__restrict__ ubl,
                                                             const float *__restrict__ S, float lo, float hi,
                                                             const km_bnd *__restrict__ bs) {
    if (bs->skip_plain) return;
    extern __shared__ float Sp[];
    __shared__ float s_min[KD_SW][64];
    __shared__ uint32_t s_arg[KD_SW][64];
    const int kpad = 32 * nchunks;
    for (int p = threadIdx.x; p < kpad; p += 64 * KD_SW) {
        const int c = km_bnd_centre(p >> 5, (p >> 4) & 1, p & 15);
        Sp[p] = c < k ? S[c] : -INFINITY;
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
    const int64_t w = blockIdx.x;
    const int64_t tile = w * tstride;
    const int64_t row = tile * 32 + (lane & 31);
    const bool real = row < n;
    const float xsq_up = real ? xsq[2 * row] : 0.0f, exn = real ? xsq[2 * row + 1] : 0.0f;
    float nx;
    const float E = km_screen_E(xsq_up, exn, maxes[0], maxes[1], maxes[2], q, nx);
    // D_c >= |x|^2 + a'_c - E; the slack 2^-21 (|x|^2 + E + max |a'|) covers the float32 additions
    const float xlo = xsq_up * (1.0f - 0x1p-18f);
    const float lbase = (xlo - E) - 0x1p-21f * (xlo + E + maxes[1] + 2.0f * nx * maxes[0] + E);
    float vmin = INFINITY;
    uint32_t vidx = 0;
    for (int ch = wave; ch < nchunks; ch += KD_SW) {
        const float4 *rp = reinterpret_cast<const float4 *>(sraw + ((w * nchunks + ch) * 64 + lane) * 16);
        const float4 r0 = rp[0], r1 = rp[1], r2 = rp[2], r3 = rp[3];
        const float a[16] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w,
                             r2.x, r2.y, r2.z, r2.w, r3.x, r3.y, r3.z, r3.w};
        uint32_t pk[8];
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
            float b[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int c = km_bnd_centre(ch, h, v + e);
                const float sc = Sp[32 * ch + 16 * h + v + e];
                if (c < k && a[v + e] < vmin) {
                    vmin = a[v + e];
                    vidx = (uint32_t)c;
                }
                const float x = (__builtin_sqrtf(fmaxf(lbase + a[v + e], 0.0f)) * lo + (sc < INFINITY ? sc : 0.0f)) *
                                (1.0f - 0x1p-22f);
                b[e] = c >= k ? 65504.0f : sc < INFINITY ? fminf(x, 65504.0f) : 0.0f;
            }
            pk[v / 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[0], b[1]));
        }
        uint4 *dst = reinterpret_cast<uint4 *>(lb + ((tile * nchunks + ch) * 64 + lane) * 16);
        dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    }
    s_min[wave][lane] = vmin;
    s_arg[wave][lane] = vidx;
    __syncthreads();
    if (wave != 0 || !real || h != 0) return;
    float m = INFINITY;
    uint32_t a = 0;
    for (int ww = 0; ww < KD_SW; ww++)
        for (int hh = 0; hh < 2; hh++) {
            const float mv = s_min[ww][lane + 32 * hh];
            const uint32_t av = s_arg[ww][lane + 32 * hh];
            if (mv < m || (mv == m && av < a)) {
                m = mv;
                a = av;
            }
        }
    float u = INFINITY;   // D_m <= |x|^2 + a'_m + E for the smallest screen value
    if (xsq_up < INFINITY && m < 3.0e38f) u = __builtin_sqrtf(fmaxf(0.0f, xsq_up + m + E) * (1.0f + 0x1p-20f)) * hi;
    ub[row] = u < INFINITY ? u : INFINITY;
    ubl[row] = a;
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

// One block: this pass's mode from the sample (see the file's head), the gates, the counters; a build begins a new
// frame (S = 0). When the loop has stopped every gate closes.
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
        int build = 0;
        if (bs->built && pays) {   // a pass on the bounds
            bs->skip_plain = 1;
            bs->skip_bscreen = 1;
            bs->skip_list = 0;
            bs->n_bounds++;
        } else {                   // a screened pass: build when the sample says bounds built now would pay
            build = (!bs->built && bs->sample_ok && pays) ? 1 : 0;
            bs->built = build;
            bs->n_builds += build;
            bs->skip_plain = build;
            bs->skip_bscreen = !build;
            bs->skip_list = 1;
        }
        bs->build = build;
        bs->sample_ok = 1;   // this pass leaves bounds for the sample tiles (the resample, a build, or the refresh)
        s_screen = build;
    }
    __syncthreads();
    if (s_screen)   // a build begins a new frame: every tile's bounds are written with S = 0
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
float km_bnd_lo(int d) { return (float)(1.0 - 2.0 * km_screen_gamma(d + 2) - 0x1p-19); }
float km_bnd_hi(int d) { return (float)(1.0 + 2.0 * km_screen_gamma(d + 2) + 0x1p-19); }

hipError_t km_launch_bnd_drift(const float *C, float *Clast, int k, int d, int valid, float *S, float *delta,
                               km_bnd *bs, const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_drift, dim3((unsigned)((k + 3) / 4)), dim3(256), 0, s, C, Clast, k, d, valid, S, delta, bs,
                       stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_count(const uint16_t *lb, const float *ub, const uint32_t *ubl, int64_t n, int k,
                               int nchunks, int64_t tstride, const float *S, const float *delta, float hi,
                               km_bnd *bs, const int32_t *stop, hipStream_t s) {
    const int64_t nwork = ((n + 31) / 32 + tstride - 1) / tstride;
    hipLaunchKernelGGL(k_bnd_count, dim3((unsigned)nwork), dim3(64 * KD_SW), (size_t)nchunks * 32 * sizeof(float), s,
                       lb, ub, ubl, n, k, nchunks, tstride, S, delta, hi, bs, stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_resample(const float *sraw, const float *xsq, int64_t n, int d, int ds, const float *maxes,
                                  int k, int nchunks, int64_t tstride, uint16_t *lb, float *ub, uint32_t *ubl,
                                  const float *S, km_bnd *bs, hipStream_t s) {
    const int64_t nwork = ((n + 31) / 32 + tstride - 1) / tstride;
    hipLaunchKernelGGL(k_bnd_resample, dim3((unsigned)nwork), dim3(64 * KD_SW),
                       (size_t)nchunks * 32 * sizeof(float), s, sraw, xsq, n, km_screen_consts(16 * ds + 2), maxes, k,
                       nchunks, tstride, lb, ub, ubl, S, km_bnd_lo(d) * (1.0f - 0x1p-21f),
                       km_bnd_hi(d) * (1.0f + 0x1p-21f), bs);
    return hipGetLastError();
}

hipError_t km_launch_bnd_decide(km_bnd *bs, double max_visited, float *S, int k, const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_decide, dim3(1), dim3(256), 0, s, bs, max_visited, S, k, stop);
    return hipGetLastError();
}

hipError_t km_launch_bnd_list(const uint16_t *lb, float *ub, const uint32_t *ubl, int64_t n, int k, int nchunks,
                              const float *S, const float *delta, float hi, uint16_t *ncand, uint16_t *cand, int slot,
                              uint32_t *over, uint32_t *multi, km_control *ctl, km_bnd *bs, int cus, hipStream_t s) {
    const int64_t nwork = (n + 31) / 32;
    const int64_t blocks = std::min<int64_t>((nwork + 3) / 4, (int64_t)cus * 4);
    hipLaunchKernelGGL(k_bnd_list, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256),
                       (size_t)nchunks * 32 * sizeof(float), s, lb, ub, ubl, n, k, nchunks, S, delta, hi, ncand, cand,
                       slot, over, multi, ctl, &bs->skip_list);
    return hipGetLastError();
}

hipError_t km_launch_bnd_overfix(const uint32_t *over, const km_control *ctl, const uint32_t *labels,
                                 const float *best, float *ub, uint32_t *ubl, float hi, const km_bnd *bs,
                                 const int32_t *stop, hipStream_t s) {
    hipLaunchKernelGGL(k_bnd_overfix, dim3(64), dim3(256), 0, s, over, ctl, labels, best, ub, ubl, hi, bs, stop);
    return hipGetLastError();
}
