// Empty-cluster relocation on the device: the reference's rule (core.py:2224-2242, scikit-learn's
// _relocate_empty_clusters) without reading the rows' distances back to the host.
//
// Each empty cluster, in ascending index, takes one of the rows farthest from their centres - ordered by best
// distance, largest first, then by row index - up to min(#empty, n) rows. A taken row leaves its old cluster
// (its sums and count are subtracted, in the order the rows are taken) and becomes its new cluster's only row.
// Centres are then sums / counts in float64, rounded to float32; a cluster with no rows left takes the centre of
// the largest cluster (the first on a tie).
//
// Selection: a best distance is non-negative (or +inf), so its bit pattern orders as the value; NaN, -0 and +0 map
// to key 0. A radix select of 11 + 11 + 10 bits finds the key T of the m-th largest row: the rows with a larger
// key are all taken, and of the rows with key T the ones with the lowest row indices (a per-block count, an
// exclusive scan over the blocks in row order, and in-block ranks). One block then orders the m taken rows and
// applies them to a float64 copy of the totals, one dimension per thread, in that order.
#include "km_internal.h"

#include <vector>

namespace {

constexpr int RL_BINS = 2048;
constexpr int RL_TB = 256;
// state words: 0 m (rows to take), 1 key prefix, 2 rows still to take at the prefix, 3 largest key,
// 4 rows with a key above T collected, 5 empty clusters; from word 16 the histogram, RL_BINS 64-bit counts (a bin
// can hold more than 2^32 rows)
enum { RL_M = 0, RL_PREFIX, RL_NEED, RL_KMAX, RL_NGT, RL_NEMPTY, RL_HIST = 16 };

__device__ __forceinline__ unsigned long long *rl_hist(uint32_t *st) {
    return reinterpret_cast<unsigned long long *>(st + RL_HIST);
}

__device__ __forceinline__ uint32_t rl_key(float b) { return b > 0.0f ? __float_as_uint(b) : 0u; }

// exclusive prefix of a 0/1 flag over a block of RL_TB threads (row order = thread order); returns the block total
__device__ __forceinline__ uint32_t rl_block_rank(bool flag, uint32_t *rank, uint32_t *s_w) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t b = __ballot(flag);
    const uint32_t below = __popcll(b & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
    __syncthreads();
    if (lane == 0) s_w[wave] = __popcll(b);
    __syncthreads();
    uint32_t off = 0, total = 0;
    for (int w = 0; w < RL_TB / 64; w++) {
        if (w < wave) off += s_w[w];
        total += s_w[w];
    }
    *rank = off + below;
    return total;
}

__global__ __launch_bounds__(1024) void k_rl_init(const double *__restrict__ tot, int k, int w, int64_t n,
                                                  uint32_t *__restrict__ st, int32_t *__restrict__ empties) {
    __shared__ uint32_t s_w[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < RL_HIST + 2 * RL_BINS; e += 1024) st[e] = 0;
    uint32_t base = 0;
    for (int c0 = 0; c0 < k; c0 += 1024) {
        const int c = c0 + tid;
        const bool empty = c < k && llrint(tot[(int64_t)c * w]) == 0;
        const uint64_t b = __ballot(empty);
        const uint32_t below = __popcll(b & ((lane == 0) ? 0ull : (~0ull >> (64 - lane))));
        __syncthreads();
        if (lane == 0) s_w[wave] = __popcll(b);
        __syncthreads();
        uint32_t off = 0, total = 0;
        for (int q = 0; q < 16; q++) {
            if (q < wave) off += s_w[q];
            total += s_w[q];
        }
        if (empty) empties[base + off + below] = c;
        base += total;
    }
    if (tid == 0) {
        const uint32_t m = (int64_t)base < n ? base : (uint32_t)n;
        st[RL_NEMPTY] = base;
        st[RL_M] = m;
        st[RL_NEED] = m;
    }
}

// Histogram of key bits [shift, shift + width) over the rows whose higher bits equal the prefix found so far.
__global__ __launch_bounds__(RL_TB) void k_rl_hist(const float *__restrict__ best, int64_t n, uint32_t *st,
                                                   int shift, int width) {
    __shared__ uint32_t h[RL_BINS];
    if (st[RL_M] == 0) return;
    for (int e = threadIdx.x; e < RL_BINS; e += RL_TB) h[e] = 0;
    __syncthreads();
    const uint32_t hm = shift + width >= 32 ? 0u : (~0u << (shift + width));
    const uint32_t pre = st[RL_PREFIX] & hm;
    const uint32_t bm = (1u << width) - 1u;
    uint32_t kmax = 0;
    for (int64_t r = (int64_t)blockIdx.x * RL_TB + threadIdx.x; r < n; r += (int64_t)gridDim.x * RL_TB) {
        const uint32_t key = rl_key(best[r]);
        kmax = key > kmax ? key : kmax;
        if ((key & hm) == pre) atomicAdd(&h[(key >> shift) & bm], 1u);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < RL_BINS; e += RL_TB)
        if (h[e]) atomicAdd(rl_hist(st) + e, (unsigned long long)h[e]);
    if (shift == 21) {
        for (int off = 32; off > 0; off >>= 1) {
            const uint32_t o = __shfl_xor(kmax, off);
            kmax = o > kmax ? o : kmax;
        }
        if ((threadIdx.x & 63) == 0) atomicMax(&st[RL_KMAX], kmax);
    }
}

// The bin holding the need-th largest remaining key: it joins the prefix, the rows above it leave the count.
__global__ __launch_bounds__(64) void k_rl_pick(uint32_t *st, int shift) {
    if (st[RL_M] == 0) return;
    if (threadIdx.x == 0) {
        const uint32_t need = st[RL_NEED];
        unsigned long long cum = 0;   // below need (at most m) until the loop stops
        int b = RL_BINS - 1;
        for (; b > 0; b--) {
            const unsigned long long h = rl_hist(st)[b];
            if (cum + h >= need) break;
            cum += h;
        }
        st[RL_PREFIX] |= (uint32_t)b << shift;
        st[RL_NEED] = need - (uint32_t)cum;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < RL_BINS; e += 64) rl_hist(st)[e] = 0;
}

// Rows with key T in each block's contiguous range.
__global__ __launch_bounds__(RL_TB) void k_rl_count(const float *__restrict__ best, int64_t n, int64_t rpb,
                                                    const uint32_t *__restrict__ st, uint32_t *__restrict__ tiecnt) {
    __shared__ uint32_t s[RL_TB / 64];
    if (st[RL_M] == 0) return;
    const uint32_t T = st[RL_PREFIX];
    const int64_t r0 = (int64_t)blockIdx.x * rpb, r1 = r0 + rpb < n ? r0 + rpb : n;
    uint32_t c = 0;
    for (int64_t r = r0 + threadIdx.x; r < r1; r += RL_TB) c += rl_key(best[r]) == T;
    for (int off = 32; off > 0; off >>= 1) c += __shfl_xor(c, off);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < RL_TB / 64; w++) t += s[w];
        tiecnt[blockIdx.x] = t;
    }
}

// Exclusive scan of the per-block tie counts, in block (row) order. An offset is only compared with the rows still
// to take (at most m < 2^32), so offsets saturate at 2^32 - 1 instead of wrapping.
__global__ __launch_bounds__(64) void k_rl_scan(uint32_t *tiecnt, int nb, const uint32_t *st) {
    if (st[RL_M] == 0) return;
    if (threadIdx.x == 0) {
        unsigned long long run = 0;
        for (int b = 0; b < nb; b++) {
            const uint32_t v = tiecnt[b];
            tiecnt[b] = run < 0xffffffffull ? (uint32_t)run : 0xffffffffu;
            run += v;
        }
    }
}

__global__ __launch_bounds__(RL_TB) void k_rl_collect(const float *__restrict__ best, int64_t n, int64_t rpb,
                                                      uint32_t *st, const uint32_t *__restrict__ tieoff,
                                                      int64_t *__restrict__ sel) {
    __shared__ uint32_t s_w[RL_TB / 64];
    const uint32_t m = st[RL_M];
    if (m == 0) return;
    const uint32_t T = st[RL_PREFIX], need = st[RL_NEED];
    const int64_t r0 = (int64_t)blockIdx.x * rpb, r1 = r0 + rpb < n ? r0 + rpb : n;
    unsigned long long run = tieoff[blockIdx.x];
    for (int64_t c0 = r0; c0 < r1; c0 += RL_TB) {   // block-uniform trip count: every thread reaches the barriers
        const int64_t r = c0 + threadIdx.x;
        const uint32_t key = r < r1 ? rl_key(best[r]) : 0u;
        const bool tie = r < r1 && key == T;
        if (r < r1 && key > T) sel[atomicAdd(&st[RL_NGT], 1u)] = r;
        uint32_t rank;
        const uint32_t total = rl_block_rank(tie, &rank, s_w);
        if (tie && run + rank < need) sel[(m - need) + run + rank] = r;
        run += total;
    }
}

struct rl_part {
    const float *X;
    int64_t row0;
};

// Orders the taken rows, applies them to a float64 copy of the totals and writes every centre.
__global__ __launch_bounds__(1024) void k_rl_apply(const uint32_t *__restrict__ st, const int64_t *__restrict__ sel,
                                                   int64_t *__restrict__ ord, const float *__restrict__ best,
                                                   const uint32_t *__restrict__ labels, const rl_part *__restrict__ parts,
                                                   int nparts, const double *__restrict__ tot, double *__restrict__ ws,
                                                   int k, int d, const int32_t *__restrict__ empties,
                                                   float *__restrict__ Cn) {
    __shared__ long long s_cnt[16];
    __shared__ int s_arg[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, w = d + 2;
    const int64_t kw = (int64_t)k * w;
    for (int64_t e = tid; e < kw; e += 1024) ws[e] = tot[e];
    const uint32_t m = (st[RL_KMAX] > 0u) ? st[RL_M] : 0u;   // every row at distance 0: nothing to move
    // order: key descending, then row ascending (the keys are distinct (key, row) pairs)
    for (uint32_t i = tid; i < m; i += 1024) {
        const int64_t ri = sel[i];
        const uint32_t ki = rl_key(best[ri]);
        uint32_t rank = 0;
        for (uint32_t j = 0; j < m; j++) {
            const int64_t rj = sel[j];
            const uint32_t kj = rl_key(best[rj]);
            rank += (kj > ki) || (kj == ki && rj < ri);
        }
        ord[rank] = ri;
    }
    __syncthreads();
    for (uint32_t t = 0; t < m; t++) {
        const int64_t f = ord[t];
        int lo = 0, hi = nparts - 1;   // the slice holding row f
        while (lo < hi) {
            const int mid = (lo + hi + 1) / 2;
            if (parts[mid].row0 <= f) lo = mid;
            else hi = mid - 1;
        }
        const float *x = parts[lo].X + (f - parts[lo].row0) * d;
        const int64_t old = labels[f], nw = empties[t];
        for (int j = tid; j < d; j += 1024) {
            const double v = (double)x[j];
            ws[old * w + 2 + j] -= v;
            ws[nw * w + 2 + j] = v;
        }
        if (tid == 0) {
            ws[old * w] -= 1.0;
            ws[nw * w] = 1.0;
        }
    }
    __syncthreads();
    // the largest cluster, the first on a tie
    long long mx = -1;
    int arg = 0;
    for (int c = tid; c < k; c += 1024) {
        const long long cnt = llrint(ws[(int64_t)c * w]);
        if (cnt > mx) { mx = cnt; arg = c; }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const long long mo = __shfl_xor(mx, off);
        const int ao = __shfl_xor(arg, off);
        if (mo > mx || (mo == mx && ao < arg)) { mx = mo; arg = ao; }
    }
    if (lane == 0) { s_cnt[wave] = mx; s_arg[wave] = arg; }
    __syncthreads();
    mx = s_cnt[0];
    arg = s_arg[0];
    for (int q = 1; q < 16; q++)
        if (s_cnt[q] > mx || (s_cnt[q] == mx && s_arg[q] < arg)) { mx = s_cnt[q]; arg = s_arg[q]; }
    const int big = arg;
    for (int64_t e = tid; e < (int64_t)k * d; e += 1024) {
        const int64_t c = e / d, j = e - c * d;
        const long long cnt = llrint(ws[c * w]);
        if (cnt > 0) Cn[e] = (float)(ws[c * w + 2 + j] / (double)cnt);
    }
    __syncthreads();
    for (int64_t e = tid; e < (int64_t)k * d; e += 1024) {
        const int64_t c = e / d, j = e - c * d;
        if (llrint(ws[c * w]) <= 0) Cn[e] = Cn[(int64_t)big * d + j];
    }
}

}  // namespace

size_t km_reloc_state_words() { return RL_HIST + 2 * RL_BINS; }
int64_t km_reloc_blocks(int64_t n, int cus) {
    int64_t nb = (n + 4095) / 4096;
    const int64_t cap = (int64_t)cus * 16;
    return nb < 1 ? 1 : (nb > cap ? cap : nb);
}

hipError_t km_launch_relocate(const double *tot, int k, int d, int64_t n, const float *best, const uint32_t *labels,
                              const float *const *part_X, const int64_t *part_rows, int nparts, void *parts_dev,
                              uint32_t *st, int32_t *empties, int64_t *sel, int64_t *ord, uint32_t *tiecnt,
                              double *ws, float *Cn, int cus, hipStream_t s) {
    if (k < 1 || d < 1 || n < 1 || nparts < 1) return hipErrorInvalidValue;
    // the slice table, through the stream (each slice's base pointer and first row)
    std::vector<rl_part> tab(nparts);
    int64_t r0 = 0;
    for (int i = 0; i < nparts; i++) {
        tab[i].X = part_X[i];
        tab[i].row0 = r0;
        r0 += part_rows[i];
    }
    if (r0 != n) return hipErrorInvalidValue;
    hipError_t e = hipMemcpyAsync(parts_dev, tab.data(), nparts * sizeof(rl_part), hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return e;
    // the copy reads the host table before the call returns
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    const int nb = (int)km_reloc_blocks(n, cus);
    int64_t rpb = (n + nb - 1) / nb;
    rpb = (rpb + RL_TB - 1) / RL_TB * RL_TB;
    const int hist_blocks = cus * 4;
    hipLaunchKernelGGL(k_rl_init, dim3(1), dim3(1024), 0, s, tot, k, d + 2, n, st, empties);
    const int passes[3][2] = {{21, 11}, {10, 11}, {0, 10}};   // (shift, width): bits 31..21, 20..10, 9..0
    for (auto &p : passes) {
        hipLaunchKernelGGL(k_rl_hist, dim3(hist_blocks), dim3(RL_TB), 0, s, best, n, st, p[0], p[1]);
        hipLaunchKernelGGL(k_rl_pick, dim3(1), dim3(64), 0, s, st, p[0]);
    }
    hipLaunchKernelGGL(k_rl_count, dim3(nb), dim3(RL_TB), 0, s, best, n, rpb, st, tiecnt);
    hipLaunchKernelGGL(k_rl_scan, dim3(1), dim3(64), 0, s, tiecnt, nb, st);
    hipLaunchKernelGGL(k_rl_collect, dim3(nb), dim3(RL_TB), 0, s, best, n, rpb, st, tiecnt, sel);
    hipLaunchKernelGGL(k_rl_apply, dim3(1), dim3(1024), 0, s, st, sel, ord, best, labels, (const rl_part *)parts_dev,
                       nparts, tot, ws, k, d, empties, Cn);
    return hipGetLastError();
}
