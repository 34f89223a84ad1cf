// Greedy k-means++ seeding on a row sample, every round on the device (the reference's kmeans_pp_init,
// mlx_kmeans/core.py:153-192, with its kernels _PP_PICK_SRC / _PP_EVAL_SRC, core.py:70-106).
//
// Round r (r = 0 .. k-2) draws `trials` = 2 + floor(ln k) candidates with probability proportional to d2, each
// row's squared distance to the nearest centre picked so far, and keeps the candidate whose picking lowers the
// sum of d2 the most:
//   k_pp_pick    candidate t of the round is the row with the largest d2_i / E_i, E_i = -ln u_i an exponential
//                variate from the counter-based hash u_i = u01(mix64(seed_r ^ mix64(i * trials + t))) (the
//                reference's Gumbel-max key ln d2 - ln(-ln u) orders rows the same way); float64 keys, the lower
//                row on an exact tie; one block per (trial, 2048-row chunk), the best of each chunk
//   k_pp_eval    the chunks' best per trial, then per row the direct-form float32 distance to each candidate
//                (dims ascending, product and add rounded separately) and min(d2, distance); per block of 32 rows
//                and trial the float64 sum of those minima in a fixed tree order. The sample is held transposed
//                (dims x m), so the reads of one dim for consecutive rows are contiguous
//   k_pp_commit  per trial the block sums added in a fixed order (64 strided running sums, then a tree); the
//                first smallest total picks the candidate; its column of minima is the next round's d2
// Nothing returns to the host until the last round; d2 lives as one column of a double-buffered (trials x m)
// array of minima, selected by the index the previous commit stored.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

static constexpr int PP_THREADS = 256;
static constexpr int PP_CHUNK = 2048;   // rows per pick block

// splitmix64's output function (the reference's mix64, core.py:43-48): a counter-based generator
__device__ __forceinline__ uint64_t pp_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// ST[c][j] = SR[j][c] = X[idx[j]][c] for the sample rows j in [j0, j1) that fall in this slice (idx local to the
// slice): the sample transposed, dims x m (a dim's rows contiguous, for the rows of an evaluation block), and as
// rows, m x dims (a row's dims contiguous, for the round's candidates)
__global__ __launch_bounds__(PP_THREADS) void k_pp_gather(const float *__restrict__ X, const int64_t *__restrict__ idx,
                                                          int64_t j0, int64_t j1, int64_t m, int d,
                                                          float *__restrict__ ST, float *__restrict__ SR) {
    const int64_t total = (j1 - j0) * d;
    for (int64_t e = (int64_t)blockIdx.x * PP_THREADS + threadIdx.x; e < total; e += (int64_t)gridDim.x * PP_THREADS) {
        const int64_t j = j0 + e / d;
        const int c = (int)(e % d);
        const float v = X[idx[j] * d + c];
        ST[(int64_t)c * m + j] = v;
        SR[j * d + c] = v;
    }
}

// |S_i - S_j|^2 of two sample rows in the direct form: dims ascending, product and add rounded separately
__device__ __forceinline__ float pp_dist(const float *__restrict__ ST, int64_t m, int d, int64_t i, int64_t j) {
    float s = 0.0f;
    for (int c = 0; c < d; c++) {
        const float q = ST[(int64_t)c * m + i] - ST[(int64_t)c * m + j];
        s = s + q * q;
    }
    return s;
}

// d2 of the first pick (stored as column 0 of the minima buffer), best index 0, picks[0] = first
__global__ __launch_bounds__(PP_THREADS) void k_pp_init(const float *__restrict__ ST, int64_t m, int d, int64_t first,
                                                        float *__restrict__ d2, uint32_t *__restrict__ best,
                                                        uint32_t *__restrict__ picks) {
    const int64_t i = (int64_t)blockIdx.x * PP_THREADS + threadIdx.x;
    if (i < m) d2[i] = pp_dist(ST, m, d, i, first);
    if (i == 0) {
        best[0] = 0;
        picks[0] = (uint32_t)first;
    }
}

// (key, row) of the better of two: larger key, lower row on a tie
__device__ __forceinline__ void pp_better(double &k, uint32_t &r, double k2, uint32_t r2) {
    if (k2 > k || (k2 == k && r2 < r)) {
        k = k2;
        r = r2;
    }
}

// block (chunk, t): the row of the chunk with the largest key for trial t
__global__ __launch_bounds__(PP_THREADS) void k_pp_pick(const float *__restrict__ mins_prev, const uint32_t *__restrict__ best,
                                                        int64_t m, int trials, uint64_t seed, double *__restrict__ ckey,
                                                        uint32_t *__restrict__ crow) {
    const float *d2 = mins_prev + (int64_t)best[0] * m;
    const int t = blockIdx.y, chunk = blockIdx.x;
    const int64_t i0 = (int64_t)chunk * PP_CHUNK, i1 = (i0 + PP_CHUNK < m) ? i0 + PP_CHUNK : m;
    double bk = -1.0;   // keys are >= 0; -1 loses to every row
    uint32_t br = 0xffffffffu;
    for (int64_t i = i0 + threadIdx.x; i < i1; i += PP_THREADS) {
        const uint64_t h = pp_mix64(seed ^ pp_mix64((uint64_t)i * (uint64_t)trials + (uint64_t)t));
        const double u = ((double)(h >> 40) + 0.5) * 0x1p-24;
        const double key = fmax((double)d2[i], 1e-30) / -log(u);
        pp_better(bk, br, key, (uint32_t)i);
    }
    __shared__ double sk[PP_THREADS];
    __shared__ uint32_t sr[PP_THREADS];
    sk[threadIdx.x] = bk;
    sr[threadIdx.x] = br;
    __syncthreads();
    for (int h = PP_THREADS / 2; h > 0; h >>= 1) {
        if (threadIdx.x < h) {
            double k = sk[threadIdx.x];
            uint32_t r = sr[threadIdx.x];
            pp_better(k, r, sk[threadIdx.x + h], sr[threadIdx.x + h]);
            sk[threadIdx.x] = k;
            sr[threadIdx.x] = r;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        ckey[t * gridDim.x + chunk] = sk[0];
        crow[t * gridDim.x + chunk] = sr[0];
    }
}

// Per (row, trial): the minimum of d2 and the distance to the trial's candidate; per block and trial the float64
// sum. A block takes PP_ROWS rows and PP_THREADS / PP_ROWS trials; the rows (from ST, a dim's 32 rows one
// 128-byte line) and the candidates (from SR, a trial's chunk of dims contiguous: from ST each candidate value
// would be a line of its own) pass through LDS PP_DCHUNK dims at a time, and each thread adds its pair's dims in
// ascending order. Rows are padded by one float so that the 32 rows of a half-wave read distinct banks.
static constexpr int PP_ROWS = 32, PP_DCHUNK = 256, PP_TPB = PP_THREADS / PP_ROWS;
__global__ __launch_bounds__(PP_THREADS) void k_pp_eval(const float *__restrict__ ST, const float *__restrict__ SR,
                                                        int64_t m, int d,
                                                        const float *__restrict__ mins_prev, const uint32_t *__restrict__ best,
                                                        const double *__restrict__ ckey, const uint32_t *__restrict__ crow,
                                                        int nchunk, int trials, float *__restrict__ mins,
                                                        double *__restrict__ part, uint32_t *__restrict__ cand) {
    const int tid = threadIdx.x, r = tid % PP_ROWS, tl = tid / PP_ROWS;
    const int t = blockIdx.y * PP_TPB + tl;   // this thread's trial
    __shared__ uint32_t sc[PP_TPB];
    __shared__ float xs[PP_ROWS][PP_DCHUNK + 1];
    __shared__ float cs[PP_TPB][PP_DCHUNK + 1];
    if (tid < PP_TPB) {
        const int tt = blockIdx.y * PP_TPB + tid;
        uint32_t rr = 0;
        if (tt < trials) {
            double k = -2.0;
            rr = 0xffffffffu;
            for (int c = 0; c < nchunk; c++) pp_better(k, rr, ckey[tt * nchunk + c], crow[tt * nchunk + c]);
            if (blockIdx.x == 0) cand[tt] = rr;
        }
        sc[tid] = rr;
    }
    const int64_t row0 = (int64_t)blockIdx.x * PP_ROWS, i = row0 + r;
    const bool live = i < m && t < trials;
    float s = 0.0f;
    for (int c0 = 0; c0 < d; c0 += PP_DCHUNK) {
        const int w = (d - c0 < PP_DCHUNK) ? d - c0 : PP_DCHUNK;
        __syncthreads();   // sc is written; the previous chunk is consumed
        // every load of the chunk in flight before the first store (fully unrolled)
        float xv[PP_ROWS * PP_DCHUNK / PP_THREADS], cv[PP_TPB * PP_DCHUNK / PP_THREADS];
#pragma unroll
        for (int q = 0; q < PP_ROWS * PP_DCHUNK / PP_THREADS; q++) {
            const int e = tid + q * PP_THREADS, c = e / PP_ROWS, rr = e % PP_ROWS;   // a dim's rows are contiguous
            xv[q] = (c < w && row0 + rr < m) ? ST[(int64_t)(c0 + c) * m + row0 + rr] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PP_TPB * PP_DCHUNK / PP_THREADS; q++) {
            const int e = tid + q * PP_THREADS, tt = e / PP_DCHUNK, c = e % PP_DCHUNK;
            cv[q] = (c < w && blockIdx.y * PP_TPB + tt < trials) ? SR[(int64_t)sc[tt] * d + c0 + c] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < PP_ROWS * PP_DCHUNK / PP_THREADS; q++) {
            const int e = tid + q * PP_THREADS;
            xs[e % PP_ROWS][e / PP_ROWS] = xv[q];
        }
#pragma unroll
        for (int q = 0; q < PP_TPB * PP_DCHUNK / PP_THREADS; q++) {
            const int e = tid + q * PP_THREADS;
            cs[e / PP_DCHUNK][e % PP_DCHUNK] = cv[q];
        }
        __syncthreads();
        if (live)
            for (int c = 0; c < w; c++) {
                const float q = xs[r][c] - cs[tl][c];
                s = s + q * q;
            }
    }
    float v = 0.0f;
    if (live) {
        v = fminf(mins_prev[(int64_t)best[0] * m + i], s);
        mins[(int64_t)t * m + i] = v;
    }
    // the block's sum for each of its trials: the 32 rows of a trial are one half-wave; a fixed halving tree
    __shared__ double ps[PP_THREADS];
    ps[tid] = (double)v;
    __syncthreads();
    for (int h = PP_ROWS / 2; h > 0; h >>= 1) {
        if (r < h) ps[tid] += ps[tid + h];
        __syncthreads();
    }
    if (r == 0 && t < trials) part[(int64_t)t * gridDim.x + blockIdx.x] = ps[tid];
}

// the round's winner: the first trial with the smallest total. Wave t adds trial t's block sums: lane l the
// blocks b = l (mod 64) in ascending order, then the 64 lane sums by a fixed halving tree.
__global__ __launch_bounds__(64 * KM_PP_MAX_TRIALS) void k_pp_commit(const double *__restrict__ part, int nblk, int trials,
                                                                     const uint32_t *__restrict__ cand,
                                                                     uint32_t *__restrict__ best,
                                                                     uint32_t *__restrict__ picks, int r) {
    __shared__ double tot[KM_PP_MAX_TRIALS];
    const int t = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (t < trials) {
        const double *p = part + (int64_t)t * nblk;
        double sum = 0.0;
        for (int b = lane; b < nblk; b += 64) sum += p[b];
        for (int h = 32; h > 0; h >>= 1) {
            const double o = __shfl_down(sum, h);
            if (lane < h) sum += o;
        }
        if (lane == 0) tot[t] = sum;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int bt = 0;
        for (int u = 1; u < trials; u++)
            if (tot[u] < tot[bt]) bt = u;
        best[0] = (uint32_t)bt;
        picks[r + 1] = cand[bt];
    }
}

// C[r] = sample row picks[r]
__global__ __launch_bounds__(PP_THREADS) void k_pp_out(const float *__restrict__ ST, int64_t m, const uint32_t *__restrict__ picks,
                                                       int k, int d, float *__restrict__ C) {
    for (int64_t e = (int64_t)blockIdx.x * PP_THREADS + threadIdx.x; e < (int64_t)k * d; e += (int64_t)gridDim.x * PP_THREADS) {
        const int r = (int)(e / d), c = (int)(e % d);
        C[e] = ST[(int64_t)c * m + picks[r]];
    }
}

int km_pp_trials(int k) { return k > 1 ? 2 + (int)log((double)k) : 1; }

// the rounds' buffers, in one workspace: two (trials x m) minima arrays, the chunks' best keys and rows, the
// blocks' sums, the candidates, the chosen trial and the picks
struct PpLayout {
    size_t mins0, mins1, ckey, crow, part, cand, best, picks, bytes;
    PpLayout(int64_t m, int k) {
        const int T = km_pp_trials(k);
        const int64_t nchunk = (m + PP_CHUNK - 1) / PP_CHUNK, nblk = (m + PP_ROWS - 1) / PP_ROWS;
        size_t o = 0;
        auto take = [&](size_t b) {
            const size_t at = o;
            o += (b + 255) / 256 * 256;
            return at;
        };
        mins0 = take((size_t)T * m * 4);
        mins1 = take((size_t)T * m * 4);
        ckey = take((size_t)T * nchunk * 8);
        crow = take((size_t)T * nchunk * 4);
        part = take((size_t)T * nblk * 8);
        cand = take((size_t)T * 4);
        best = take(4);
        picks = take((size_t)k * 4);
        bytes = o;
    }
};

size_t km_pp_workspace(int64_t m, int k) { return PpLayout(m, k).bytes; }

hipError_t km_launch_pp_gather(const float *X, const int64_t *idx, int64_t j0, int64_t j1, int64_t m, int d,
                               float *ST, float *SR, hipStream_t s) {
    if (j1 <= j0) return hipSuccess;
    const int64_t total = (j1 - j0) * d;
    const int64_t blocks = (total + PP_THREADS - 1) / PP_THREADS;
    hipLaunchKernelGGL(k_pp_gather, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(PP_THREADS), 0, s, X, idx,
                       j0, j1, m, d, ST, SR);
    return hipGetLastError();
}

hipError_t km_launch_pp(const float *ST, const float *SR, int64_t m, int d, int k, int64_t first,
                        const uint64_t *seeds_h, void *ws, float *C, hipStream_t s) {
    const int T = km_pp_trials(k);
    if (T > KM_PP_MAX_TRIALS) return hipErrorInvalidValue;
    const int nchunk = (int)((m + PP_CHUNK - 1) / PP_CHUNK), nblk = (int)((m + PP_ROWS - 1) / PP_ROWS);
    const int ninit = (int)((m + PP_THREADS - 1) / PP_THREADS);
    const PpLayout L(m, k);   // the caller sized ws with km_pp_workspace
    char *w = static_cast<char *>(ws);
    float *mins[2] = {reinterpret_cast<float *>(w + L.mins0), reinterpret_cast<float *>(w + L.mins1)};
    double *ckey = reinterpret_cast<double *>(w + L.ckey);
    uint32_t *crow = reinterpret_cast<uint32_t *>(w + L.crow);
    double *part = reinterpret_cast<double *>(w + L.part);
    uint32_t *cand = reinterpret_cast<uint32_t *>(w + L.cand);
    uint32_t *best = reinterpret_cast<uint32_t *>(w + L.best);
    uint32_t *picks = reinterpret_cast<uint32_t *>(w + L.picks);
    hipLaunchKernelGGL(k_pp_init, dim3(ninit), dim3(PP_THREADS), 0, s, ST, m, d, first, mins[1], best, picks);
    hipError_t e = hipGetLastError();
    for (int r = 0; r < k - 1 && e == hipSuccess; r++) {
        const float *prev = mins[(r + 1) & 1];
        float *cur = mins[r & 1];
        hipLaunchKernelGGL(k_pp_pick, dim3(nchunk, T), dim3(PP_THREADS), 0, s, prev, best, m, T, seeds_h[r], ckey,
                           crow);
        hipLaunchKernelGGL(k_pp_eval, dim3(nblk, (T + PP_TPB - 1) / PP_TPB), dim3(PP_THREADS), 0, s, ST, SR, m, d, prev, best,
                           ckey, crow, nchunk, T, cur, part, cand);
        hipLaunchKernelGGL(k_pp_commit, dim3(1), dim3(64 * T), 0, s, part, nblk, T, cand, best, picks, r);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    const int64_t total = (int64_t)k * d;
    const int64_t blocks = (total + PP_THREADS - 1) / PP_THREADS;
    hipLaunchKernelGGL(k_pp_out, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(PP_THREADS), 0, s, ST, m, picks,
                       k, d, C);
    return hipGetLastError();
}
