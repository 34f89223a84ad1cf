// Change-only accumulation for the wide-row path's fit loop.
//
// After the pass that records every row's label, a pass of the fit loop may add to the previous pass's float64
// totals only the rows whose label changed: +x and +1 for the new cluster, -x and -1 for the old one. The rows
// that changed are listed in row order over all slices (per-block counts, an exclusive scan over the blocks,
// in-block ranks), each giving two entries (its new label with +row, its old label with -row); the entries are
// sorted by label with the counting sort of the full accumulation (stable: entry order within a label), and the
// sorted entries are added in fixed chunks of 64, one wave each, in float64 (km_chunks.hip). A pass then reads
// only the changed rows instead of every row.
//
// Each pass chooses on the device: the scan of the counts compares the number of changed rows m with a limit set
// by the host (up to which sorting 2 limit entries and reading 2m rows costs less than the full accumulation) and
// writes two gate words, one that stops the change-only kernels and one that stops the full accumulation's. Both
// are queued; exactly one runs. The finish reads the same word to know which kind of sums it was given.
//
// The inertia of a change-only pass cannot come from the rows' distances, which it no longer reads. It is formed
// from the totals in coordinates centred on the rows' mean mu: sum_c sum_{i in c} |x_i - c|^2 = T + sum_c (n_c
// |D_c|^2 - 2 D_c . (S_c - n_c mu)), with D_c = c - mu, S_c the cluster's coordinate sum and T = sum_i |x_i - mu|^2,
// all in float64 (the finish computes the per-cluster terms, KM_FIN_CENTRED). Centring keeps the cancellation to the
// ratio T / inertia, whatever the data's offset from the origin. mu and T are computed once per data set here.
#include "km_internal.h"

namespace {

constexpr int WD_RB = 4096;   // rows per block of the change count and the entry list
constexpr int WD_SB = 512;    // rows per block of the mean and scatter

// Block b of rows [b WD_SB, ...) of one slice: mode 0 the float64 column sums into part[b][0 .. d); mode 1 the
// block's sum of (x - mu)^2 into part[b][d]. With d <= 256 the block's threads form G = 256 / d row groups of d
// threads (group g takes rows g, g + G, ...), otherwise one group whose threads take dims j, j + 256, ...; the
// groups' sums are added in group order, mode 1's per-thread sums by a fixed tree.
__global__ __launch_bounds__(256) void k_wd_stats(const float *__restrict__ X, int64_t n, int d, int mode,
                                                  const double *__restrict__ mu, double *__restrict__ part) {
    __shared__ double red[256];
    const int64_t r0 = (int64_t)blockIdx.x * WD_SB;
    const int64_t r1 = r0 + WD_SB < n ? r0 + WD_SB : n;
    double *out = part + (int64_t)blockIdx.x * (d + 1);
    const int G = d <= 256 ? 256 / d : 1;
    const int g = d <= 256 ? threadIdx.x / d : 0;
    const int j0 = d <= 256 ? threadIdx.x % d : threadIdx.x;
    double q = 0.0;
    if (g < G) {
        for (int j = j0; j < d; j += (d <= 256 ? d : 256)) {
            double s = 0.0;
            const double m = mode ? mu[j] : 0.0;
            for (int64_t r = r0 + g; r < r1; r += G) {
                const double v = (double)X[r * d + j];
                if (mode) {
                    const double t = v - m;
                    s += t * t;
                } else {
                    s += v;
                }
            }
            if (mode) q += s;
            else red[threadIdx.x] = s;   // d <= 256: one dim per thread; d > 256: written below per dim
            if (!mode && d > 256) out[j] = s;
        }
    }
    if (!mode) {
        if (d > 256) return;
        __syncthreads();
        if (threadIdx.x < d) {
            double s = 0.0;
            for (int gg = 0; gg < G; gg++) s += red[gg * d + threadIdx.x];
            out[threadIdx.x] = s;
        }
        return;
    }
    red[threadIdx.x] = q;
    __syncthreads();
    for (int h = 128; h > 0; h >>= 1) {
        if (threadIdx.x < h) red[threadIdx.x] += red[threadIdx.x + h];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[d] = red[0];
}

// mode 0 (a block per 64 dims): mu[j] = the blocks' column sums / n, each dim's sum taken as four interleaved
// runs over the blocks added in run order; mode 1 (one block): mu[d] = T, the blocks' scatter as 256 interleaved
// runs added by a fixed tree. Fixed orders: the same bits every time.
__global__ __launch_bounds__(256) void k_wd_stats_fin(const double *__restrict__ part, int64_t nb, int d, int64_t n,
                                                      int mode, double *__restrict__ mu) {
    __shared__ double red[256];
    const int tid = threadIdx.x;
    if (mode) {
        double t = 0.0;
        for (int64_t b = tid; b < nb; b += 256) t += part[b * (d + 1) + d];
        red[tid] = t;
        __syncthreads();
        for (int h = 128; h > 0; h >>= 1) {
            if (tid < h) red[tid] += red[tid + h];
            __syncthreads();
        }
        if (tid == 0) mu[d] = red[0];
        return;
    }
    const int j = blockIdx.x * 64 + (tid & 63), g = tid >> 6;
    double sj = 0.0;
    if (j < d)
        for (int64_t b = g; b < nb; b += 4) sj += part[b * (d + 1) + j];
    red[tid] = sj;
    __syncthreads();
    if (g == 0 && j < d) mu[j] = (((red[tid] + red[tid + 64]) + red[tid + 128]) + red[tid + 192]) / (double)n;
}

// Rows whose label changed, per block of WD_RB rows.
__global__ __launch_bounds__(256) void k_wd_count(const uint32_t *__restrict__ lab, const uint32_t *__restrict__ prev,
                                                  int64_t n, uint32_t *__restrict__ bcnt,
                                                  const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    __shared__ uint32_t s[4];
    const int64_t r0 = (int64_t)blockIdx.x * WD_RB;
    const int64_t r1 = r0 + WD_RB < n ? r0 + WD_RB : n;
    uint32_t c = 0;
    for (int64_t r = r0 + threadIdx.x; r < r1; r += 256) c += lab[r] != prev[r];
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) bcnt[blockIdx.x] = s[0] + s[1] + s[2] + s[3];
}

// Exclusive scan of the block counts in block order (thread t scans its own run of blocks, the runs' totals are
// scanned across the threads), m into bcnt[nb], and the gate words: gate[0] = stop or m > limit (the change-only
// kernels stand down), gate[1] = stop or m <= limit (the full accumulation stands down). Runs even when stopped,
// so that the gates always hold this pass's decision.
__global__ __launch_bounds__(1024) void k_wd_scan(uint32_t *__restrict__ bcnt, int nb, int64_t limit,
                                                  int32_t *__restrict__ gate, const int32_t *__restrict__ stop) {
    __shared__ uint32_t run[1024];
    const bool stopped = stop && *stop;
    const int per = (nb + 1023) / 1024;
    const int b0 = threadIdx.x * per, b1 = min(nb, b0 + per);
    uint32_t t = 0;
    if (!stopped)
        for (int b = b0; b < b1; b++) t += bcnt[b];
    run[threadIdx.x] = t;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {   // inclusive scan of the runs' totals
        const uint32_t v = threadIdx.x >= off ? run[threadIdx.x - off] : 0u;
        __syncthreads();
        run[threadIdx.x] += v;
        __syncthreads();
    }
    const uint32_t m = run[1023];
    if (!stopped) {
        uint32_t acc = run[threadIdx.x] - t;
        for (int b = b0; b < b1; b++) {
            const uint32_t v = bcnt[b];
            bcnt[b] = acc;
            acc += v;
        }
    }
    if (threadIdx.x == 0) {
        if (!stopped) bcnt[nb] = m;
        const bool delta = !stopped && (int64_t)m <= limit;
        gate[0] = delta ? 0 : 1;
        gate[1] = (stopped || delta) ? 1 : 0;
    }
}

__device__ __forceinline__ uint32_t wd_rank(bool flag, uint32_t *s_w, uint32_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t b = __ballot(flag);
    const uint32_t below = __popcll(b & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    __syncthreads();
    if (lane == 0) s_w[wave] = __popcll(b);
    __syncthreads();
    uint32_t off = 0, tot = 0;
    for (int w = 0; w < 4; w++) {
        if (w < wave) off += s_w[w];
        tot += s_w[w];
    }
    *total = tot;
    return off + below;
}

// The changed rows in row order: entry e < m is (new label, row), entry m + e (old label, row with the top bit
// set). Runs only when the gate chose the change-only sums, so m is within the limit the entry arrays are sized for.
__global__ __launch_bounds__(256) void k_wd_write(const uint32_t *__restrict__ lab, const uint32_t *__restrict__ prev,
                                                  int64_t n, const uint32_t *__restrict__ boff, int nb,
                                                  uint32_t *__restrict__ elab, uint32_t *__restrict__ erow,
                                                  const int32_t *__restrict__ gate) {
    if (*gate) return;
    __shared__ uint32_t s_w[4];
    const uint32_t m = boff[nb];
    const int64_t r0 = (int64_t)blockIdx.x * WD_RB;
    const int64_t r1 = r0 + WD_RB < n ? r0 + WD_RB : n;
    uint32_t run = boff[blockIdx.x];
    for (int64_t c0 = r0; c0 < r1; c0 += 256) {   // block-uniform trip count: every thread reaches the barriers
        const int64_t r = c0 + threadIdx.x;
        const uint32_t nl = r < r1 ? lab[r] : 0u, ol = r < r1 ? prev[r] : 0u;
        const bool moved = r < r1 && nl != ol;
        uint32_t total;
        const uint32_t rank = wd_rank(moved, s_w, &total);
        if (moved) {
            const uint32_t e = run + rank;
            elab[e] = nl;
            erow[e] = (uint32_t)r;
            elab[m + e] = ol;
            erow[m + e] = (uint32_t)r | 0x80000000u;
        }
        run += total;
    }
}

}  // namespace

int64_t km_wd_blocks(int64_t n) { return (n + WD_RB - 1) / WD_RB; }
int64_t km_wd_stat_blocks(int64_t n) { return (n + WD_SB - 1) / WD_SB; }
int km_wd_max_dims() { return KM_CHUNK_MAX_DIMS; }

hipError_t km_launch_wd_stats(const km_slice *slices_h, const int64_t *rows, int nslices, int d, double *part,
                              double *mu_T, hipStream_t s) {
    if (d < 1 || nslices < 1) return hipErrorInvalidValue;
    int64_t n = 0, nbt = 0;
    for (int i = 0; i < nslices; i++) {
        n += rows[i];
        nbt += km_wd_stat_blocks(rows[i]);
    }
    for (int mode = 0; mode < 2; mode++) {
        int64_t b0 = 0;
        for (int i = 0; i < nslices; i++) {
            const int64_t nb = km_wd_stat_blocks(rows[i]);
            hipLaunchKernelGGL(k_wd_stats, dim3((unsigned)nb), dim3(256), 0, s, slices_h[i].X, rows[i], d, mode, mu_T,
                               part + b0 * (d + 1));
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            b0 += nb;
        }
        hipLaunchKernelGGL(k_wd_stats_fin, dim3(mode ? 1 : (d + 63) / 64), dim3(256), 0, s, part, nbt, d, n, mode, mu_T);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t km_launch_wd_gate(const uint32_t *lab, const uint32_t *prev, int64_t n, int64_t limit, uint32_t *bcnt,
                             int32_t *gate, const int32_t *stop, hipStream_t s) {
    if (n < 1 || n > (int64_t)0x7fffffff) return hipErrorInvalidValue;
    const int nb = (int)km_wd_blocks(n);
    hipLaunchKernelGGL(k_wd_count, dim3(nb), dim3(256), 0, s, lab, prev, n, bcnt, stop);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_wd_scan, dim3(1), dim3(1024), 0, s, bcnt, nb, limit, gate, stop);
    return hipGetLastError();
}

hipError_t km_launch_wd_accum(const km_slice *slices_d, int nslices, int64_t n, int d, const uint32_t *lab,
                              const uint32_t *prev, int k, int64_t limit, const uint32_t *bcnt, uint32_t *elab,
                              uint32_t *erow, uint32_t *H, uint32_t *counts, uint32_t *base, uint32_t *perm,
                              double *pieces, double *tmp, const int32_t *gate, hipStream_t s) {
    if (d < 1 || d > KM_CHUNK_MAX_DIMS || n < 1 || n > (int64_t)0x7fffffff || nslices < 1 || limit < 1 || limit > n)
        return hipErrorInvalidValue;
    const int nb = (int)km_wd_blocks(n);
    const int64_t len = 2 * limit;
    hipLaunchKernelGGL(k_wd_write, dim3(nb), dim3(256), 0, s, lab, prev, n, bcnt, nb, elab, erow, gate);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // the sort takes the 2m entries written (m on the device), not the 2 limit the arrays hold
    if ((e = km_launch_label_sort(elab, len, k, H, counts, base, perm, gate, s, bcnt + nb)) != hipSuccess) return e;
    return km_launch_chunk_sums(2, nullptr, slices_d, nslices, d, elab, erow, nullptr, nullptr, perm, counts, base, k,
                                bcnt + nb, len, pieces, tmp, gate, s);
}
