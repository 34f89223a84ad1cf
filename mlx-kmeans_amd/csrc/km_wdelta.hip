// Change-only accumulation for the wide-row path's fit loop.
//
// After the pass that records every row's label, a pass of the fit loop may add to the previous pass's float64
// totals only the rows whose label changed: +x and +1 for the new cluster, -x and -1 for the old one. The rows
// that changed are listed in row order over all slices (per-block counts, an exclusive scan over the blocks,
// in-block ranks), each giving two entries (its new label with +row, its old label with -row); the entries are
// sorted by label with the counting sort of the full accumulation (stable: entry order within a label), and the
// sorted entries are added in fixed chunks of 64, one wave each, lanes owning dims, in float64, the clusters that
// span chunks combined from per-chunk pieces in chunk order. A pass then reads only the changed rows instead of
// every row.
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
constexpr int WD_Q = 64;      // sorted entries per wave of the change sums
constexpr int WD_MAXJ = 13;   // dims per lane in the change sums: d <= 832

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

// mode 0: mu[j] = (the blocks' column sums in block order) / n; mode 1: mu[d] = T, the blocks' scatter in order.
__global__ __launch_bounds__(256) void k_wd_stats_fin(const double *__restrict__ part, int64_t nb, int d, int64_t n,
                                                      int mode, double *__restrict__ mu) {
    if (mode) {
        if (threadIdx.x == 0) {
            double t = 0.0;
            for (int64_t b = 0; b < nb; b++) t += part[b * (d + 1) + d];
            mu[d] = t;
        }
        return;
    }
    for (int j = threadIdx.x; j < d; j += 256) {
        double s = 0.0;
        for (int64_t b = 0; b < nb; b++) s += part[b * (d + 1) + j];
        mu[j] = s / (double)n;
    }
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

// Entries 2m .. 2 limit - 1 take the label k, which no cluster block reads: the sort then runs over a size the
// host knows.
__global__ __launch_bounds__(256) void k_wd_pad(uint32_t *__restrict__ elab, int64_t len, const uint32_t *__restrict__ mcount,
                                                uint32_t k, const int32_t *__restrict__ gate) {
    if (*gate) return;
    const int64_t e0 = 2 * (int64_t)*mcount;
    for (int64_t e = e0 + (int64_t)blockIdx.x * 256 + threadIdx.x; e < len; e += (int64_t)gridDim.x * 256) elab[e] = k;
}

typedef __attribute__((address_space(1))) float gfloat;

// A row's address from its entry (the slice table lists ascending first rows).
__device__ __forceinline__ const float *wd_row(const km_slice *__restrict__ slices, int nslices, int d, uint32_t er) {
    const int64_t r = (int64_t)(er & 0x7fffffffu);
    int s = 0;
    while (s + 1 < nslices && slices[s + 1].row0 <= r) s++;
    return slices[s].X + (r - slices[s].row0) * d;
}

// The change sums over the sorted entries in chunks of WD_Q: wave q takes sorted positions [q WD_Q, (q + 1) WD_Q) of
// the 2m valid ones (each cluster's run is contiguous, in entry order), loads their row addresses lane-parallel,
// then adds the rows in position order, four in flight, into float64 sums (lane owns dims lane, lane + 64, ...),
// closing a piece at every change of cluster. A cluster whose run lies inside the chunk is complete: written to tmp
// as [count, 0, x]. A cluster that runs past the chunk's edge leaves a piece: the head slot of the chunk for the
// cluster holding its first position, the tail slot for the one holding its last. Every wave does the same amount
// of work, however unevenly the changed rows fall among the clusters.
__global__ __launch_bounds__(256) void k_wd_chunks(const km_slice *__restrict__ slices, int nslices, int d,
                                                   const uint32_t *__restrict__ elab, const uint32_t *__restrict__ erow,
                                                   const uint32_t *__restrict__ perm,
                                                   const uint32_t *__restrict__ counts,
                                                   const uint32_t *__restrict__ base,
                                                   const uint32_t *__restrict__ mcount, double *__restrict__ pieces,
                                                   double *__restrict__ tmp, const int32_t *__restrict__ gate) {
    if (*gate) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t q = (int64_t)blockIdx.x * 4 + wave;
    const int64_t E = 2 * (int64_t)*mcount;
    const int64_t e0 = q * WD_Q;
    if (e0 >= E) return;   // whole waves leave; the kernel has no barriers
    const int ne = (int)(E - e0 < WD_Q ? E - e0 : WD_Q);
    // lane L: sorted position e0 + L
    uint32_t my_lab = 0xffffffffu, my_er = 0;
    if (lane < ne) {
        const uint32_t pe = perm[e0 + lane];
        my_lab = elab[pe];
        my_er = erow[pe];
    }
    const float *my_x = lane < ne ? wd_row(slices, nslices, d, my_er) : slices[0].X;
    const uint64_t my_xa = (uint64_t)(uintptr_t)my_x;
    const int W = d + 2;
    const int64_t e1 = e0 + ne;
    double acc[WD_MAXJ];
#pragma unroll
    for (int i = 0; i < WD_MAXJ; i++) acc[i] = 0.0;
    double cntd = 0.0;
    uint32_t cur = (uint32_t)__shfl((int)my_lab, 0);
    auto flush = [&](uint32_t cl) {
        const int64_t b = base[cl], e = b + counts[cl];
        double *dst;
        if (b >= e0 && e <= e1) {   // complete within the chunk
            dst = tmp + (int64_t)cl * W;
            if (lane == 0) {
                dst[0] = cntd;
                dst[1] = 0.0;
            }
            dst += 2;
        } else {
            dst = pieces + (q * 2 + (b <= e0 ? 0 : 1)) * (int64_t)(d + 1);
            if (lane == 0) dst[d] = cntd;
        }
#pragma unroll
        for (int i = 0; i < WD_MAXJ; i++) {
            const int j = lane + 64 * i;
            if (j < d) dst[j] = acc[i];
            acc[i] = 0.0;
        }
        cntd = 0.0;
    };
    for (int t = 0; t < ne; t += 4) {
        // the loads are unconditional (a lane past the last dim reads dim d - 1, a slot past the chunk's end reads
        // row t again) and masked afterwards: guarded loads become one branch and one wait each
        const gfloat *x[4];   // global address space: global loads, not flat ones
#pragma unroll
        for (int u = 0; u < 4; u++)
            x[u] = (const gfloat *)(uintptr_t)(uint64_t)__shfl((long long)my_xa, t + u < ne ? t + u : t);
        float v[4][WD_MAXJ];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int i = 0; i < WD_MAXJ; i++) v[u][i] = x[u][min(lane + 64 * i, d - 1)];
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
            for (int i = 0; i < WD_MAXJ; i++)
                if (t + u >= ne || lane + 64 * i >= d) v[u][i] = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            if (t + u >= ne) break;
            const uint32_t lb = (uint32_t)__shfl((int)my_lab, t + u);
            const bool neg = ((uint32_t)__shfl((int)my_er, t + u) >> 31) != 0;
            if (lb != cur) {
                flush(cur);
                cur = lb;
            }
#pragma unroll
            for (int i = 0; i < WD_MAXJ; i++) acc[i] = neg ? acc[i] - (double)v[u][i] : acc[i] + (double)v[u][i];
            cntd += neg ? -1.0 : 1.0;
        }
    }
    flush(cur);
}

// Block per cluster: a cluster with no changed rows gets zero change; one whose run spans several chunks the sum
// of its pieces in chunk order (the head slot of every chunk whose first position it holds, the tail slot of the
// chunk it starts in otherwise); one inside a single chunk was written whole by that chunk's wave.
__global__ __launch_bounds__(256) void k_wd_combine(const uint32_t *__restrict__ counts,
                                                    const uint32_t *__restrict__ base, int d,
                                                    const double *__restrict__ pieces, double *__restrict__ tmp,
                                                    const int32_t *__restrict__ gate) {
    if (*gate) return;
    const int c = blockIdx.x, W = d + 2;
    const int64_t cnt = counts[c], b = base[c];
    double *dst = tmp + (int64_t)c * W;
    if (cnt == 0) {
        for (int j = threadIdx.x; j < W; j += 256) dst[j] = 0.0;
        return;
    }
    const int64_t q0 = b / WD_Q, q1 = (b + cnt - 1) / WD_Q;
    if (q0 == q1) return;
    for (int j = threadIdx.x; j <= d; j += 256) {
        double t = 0.0;
        for (int64_t qa = q0; qa <= q1; qa += 8) {   // eight loads in flight, added in chunk order
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int64_t q = qa + u;
                v[u] = q <= q1 ? pieces[(q * 2 + (b <= q * WD_Q ? 0 : 1)) * (int64_t)(d + 1) + j] : 0.0;
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (qa + u <= q1) t += v[u];
        }
        if (j < d) dst[2 + j] = t;
        else dst[0] = t;
    }
    if (threadIdx.x == 0) dst[1] = 0.0;
}

}  // namespace

int64_t km_wd_blocks(int64_t n) { return (n + WD_RB - 1) / WD_RB; }
int64_t km_wd_stat_blocks(int64_t n) { return (n + WD_SB - 1) / WD_SB; }
int km_wd_max_dims() { return 64 * WD_MAXJ; }

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
        hipLaunchKernelGGL(k_wd_stats_fin, dim3(1), dim3(256), 0, s, part, nbt, d, n, mode, mu_T);
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

int64_t km_wd_piece_doubles(int64_t limit, int d) { return (2 * limit + WD_Q - 1) / WD_Q * 2 * (int64_t)(d + 1); }

hipError_t km_launch_wd_accum(const km_slice *slices_d, int nslices, int64_t n, int d, const uint32_t *lab,
                              const uint32_t *prev, int k, int64_t limit, const uint32_t *bcnt, uint32_t *elab,
                              uint32_t *erow, uint32_t *H, uint32_t *counts, uint32_t *base, uint32_t *perm,
                              double *pieces, double *tmp, const int32_t *gate, hipStream_t s) {
    if (d < 1 || d > 64 * WD_MAXJ || n < 1 || n > (int64_t)0x7fffffff || nslices < 1 || limit < 1 || limit > n)
        return hipErrorInvalidValue;
    const int nb = (int)km_wd_blocks(n);
    const int64_t len = 2 * limit;
    hipLaunchKernelGGL(k_wd_write, dim3(nb), dim3(256), 0, s, lab, prev, n, bcnt, nb, elab, erow, gate);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_wd_pad, dim3((unsigned)std::min<int64_t>((len + 255) / 256, 2048)), dim3(256), 0, s, elab, len,
                       bcnt + nb, (uint32_t)k, gate);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if ((e = km_launch_label_sort(elab, len, k + 1, H, counts, base, perm, gate, s)) != hipSuccess) return e;
    const int64_t nq = (len + WD_Q - 1) / WD_Q;
    hipLaunchKernelGGL(k_wd_chunks, dim3((unsigned)((nq + 3) / 4)), dim3(256), 0, s, slices_d, nslices, d, elab, erow,
                       perm, counts, base, bcnt + nb, pieces, tmp, gate);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_wd_combine, dim3(k), dim3(256), 0, s, counts, base, d, pieces, tmp, gate);
    return hipGetLastError();
}
