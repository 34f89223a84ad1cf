// Generic kernels of the exact Lloyd pass: they serve every (rows, dims, k) and define the semantics that the
// faster paths reproduce bit for bit.
//
//   k_assign_rows     exact nearest centre, one row per lane, direct form over every centre
//                     (reference: mlx_kmeans/core.py:263-274, the rows loop)
//   k_accum_generic   deterministic compensated per-cluster [count, best, x] into per-row-block partials
//                     (reference: the accumulation paths of core.py:1292-1466; Neumaier add of core.py:244-247)
//   k_reduce_split    partials -> float64 sums of fixed contiguous ranges of row-blocks
//   k_finish          totals, new centres (core.py:2238-2242), spherical renormalisation (estimator.py:127-130),
//                     and in its last block the counts, inertia, empties, argmax and stopping rule
//                     (core.py:2222-2242, estimator.py:147-149)
//   k_normalise       spherical renormalisation of host-given centres (the start of a fit, after a relocation)
//
// The file is compiled with -ffp-contract=off: `s + t * t` stays a separately rounded product and add.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

const char *const km_kernel_names[KK_COUNT] = {
    "km_assign_rows", "km_accum_generic", "km_reduce",     "km_finish",    "km_normalise",
    "km_fused_lowd",  "km_fused_mfma",    "km_big_prep",   "km_big_screen", "km_big_rescore",
    "km_big_accum",   "km_seed_pp",       "km_relocate",
    "km_change_sums", "km_bounds",      "km_bounds_list", "km_big_screen_bnd", "km_bounds_sample"};

// Neumaier's compensated add, the reference's KAHAN_ADD (core.py:244-247): t = s + v; the rounding error of
// that add goes to c; the true running sum is s + c.
__device__ __forceinline__ void neumaier(float &s, float &c, float v) {
    float t = s + v;
    c += (fabsf(s) >= fabsf(v)) ? ((s - t) + v) : ((v - t) + s);
    s = t;
}

// ------------------------------------------------------------------ exact assignment, one row per lane

template <int D>
__global__ __launch_bounds__(256) void k_assign_rows(const float *__restrict__ X, int64_t n, int d_rt,
                                                     const float *__restrict__ C, int k,
                                                     uint32_t *__restrict__ labels, float *__restrict__ best,
                                                     const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float bst = INFINITY;
    uint32_t bl = 0;
    if constexpr (D > 0) {
        const float *x = X + i * D;
        float xv[D];
#pragma unroll
        for (int j = 0; j < D; j++) xv[j] = x[j];
        for (int c = 0; c < k; c++) {
            const float *cc = C + (size_t)c * D;
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < D; j++) {
                float t = xv[j] - cc[j];
                s = s + t * t;
            }
            if (s < bst) { bst = s; bl = (uint32_t)c; }
        }
    } else {
        const int d = d_rt;
        const float *x = X + i * d;
        for (int c = 0; c < k; c++) {
            const float *cc = C + (size_t)c * d;
            float s = 0.0f;
            for (int j = 0; j < d; j++) {
                float t = x[j] - cc[j];
                s = s + t * t;
            }
            if (s < bst) { bst = s; bl = (uint32_t)c; }
        }
    }
    if (labels) labels[i] = bl;
    if (best) best[i] = bst;
}

// Rows wider than the register-held cases below, against four or more centres, take the tiled form of the same
// loop (km_big.hip), whose 64 x 64 tiles read each row and centre once per 32-dim step instead of every lane
// re-reading its row from the caches for every centre. Measured on MI355X, ns per row per pass (one row per lane ->
// tiled): 256 dims 11.8 -> 10.1 at 2 centres, 75 -> 5.3 at 64, 1124 -> 25 at 1024; 3072 dims 199 -> 201 at 2,
// 170 -> 111 at 8, 10510 -> 435 at 1024; at 64 dims (a register-held case) 5.3 -> 6.4 at 1024.
static constexpr int KM_TILED_MIN_DIMS = 65;
static constexpr int KM_TILED_MIN_K = 4;

hipError_t km_launch_assign_rows(const float *X, int64_t n, int d, const float *C, int k, uint32_t *labels,
                                 float *best, const int32_t *stop, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (d >= KM_TILED_MIN_DIMS && k >= KM_TILED_MIN_K && n <= (int64_t)0xffffffffu - 64)
        return km_launch_rows_tiled(X, n, d, C, k, labels, best, stop, s);
    dim3 grid((unsigned)((n + 255) / 256)), block(256);
#define KM_ROWS_CASE(DD) \
    case DD: hipLaunchKernelGGL(k_assign_rows<DD>, grid, block, 0, s, X, n, d, C, k, labels, best, stop); break;
    switch (d) {
        KM_ROWS_CASE(1) KM_ROWS_CASE(2) KM_ROWS_CASE(3) KM_ROWS_CASE(4) KM_ROWS_CASE(5) KM_ROWS_CASE(6)
        KM_ROWS_CASE(7) KM_ROWS_CASE(8) KM_ROWS_CASE(10) KM_ROWS_CASE(12) KM_ROWS_CASE(16) KM_ROWS_CASE(24)
        KM_ROWS_CASE(32) KM_ROWS_CASE(48) KM_ROWS_CASE(64)
        default: hipLaunchKernelGGL(k_assign_rows<0>, grid, block, 0, s, X, n, d, C, k, labels, best, stop);
    }
#undef KM_ROWS_CASE
    return hipGetLastError();
}

// ------------------------------------------------------------------ generic deterministic accumulation
//
// Grid: x = row-block, y = cluster-block, z = column-block; 256 threads. Columns of a cluster are
// [count, best, x_0, ..., x_{d-1}] (w = d + 2). The block scans its rows in ascending order, 256 at a time,
// and keeps the rows whose label falls in its cluster range, in ascending order. Those rows are dealt to P
// "slots" in turn (entry q of a chunk to slot q % P); a slot is DL threads, one column each, and has its own
// LDS accumulator copy, so every accumulator has exactly one writer and a fixed order of adds. At the end
// the copies are folded in slot order and written as this row-block's partial: a sum and a compensation.
// The result depends only on the data and the plan, never on scheduling.

static int next_pow2(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

static constexpr size_t KM_ACC_LDS_BUDGET = 48 * 1024;

km_accum_plan km_plan_accum_generic(int64_t n, int d, int k, int64_t max_rb) {
    km_accum_plan pl{};
    const int w = d + 2;
    pl.wb = w < 2048 ? w : 2048;
    pl.nwb = (w + pl.wb - 1) / pl.wb;
    const int dl = next_pow2(pl.wb < 256 ? pl.wb : 256);
    const int P = 256 / dl;
    int cb = (int)(KM_ACC_LDS_BUDGET / 8 / ((size_t)P * pl.wb));
    if (cb < 1) cb = 1;
    if (cb > k) cb = k;
    pl.cb = cb;
    pl.ncb = (k + cb - 1) / cb;
    // enough blocks to fill the chip several times over, but row-blocks of at least 2048 rows
    int64_t target_rb = (2048 + (int64_t)pl.ncb * pl.nwb - 1) / ((int64_t)pl.ncb * pl.nwb);
    if (target_rb < 1) target_rb = 1;
    int64_t rbs = (n + target_rb - 1) / target_rb;
    if (rbs < 2048) rbs = 2048;
    if (max_rb > 0 && (n + rbs - 1) / rbs > max_rb) rbs = (n + max_rb - 1) / max_rb;
    rbs = (rbs + 255) / 256 * 256;
    pl.rbs = rbs;
    pl.nrb = (int)((n + rbs - 1) / rbs);
    if (pl.nrb < 1) pl.nrb = 1;
    pl.lds = (size_t)P * cb * pl.wb * 2 * sizeof(float) + (256 + 8) * sizeof(int);
    return pl;
}

__global__ __launch_bounds__(256) void k_accum_generic(const float *__restrict__ X, int64_t n, int d,
                                                       const uint32_t *__restrict__ labels,
                                                       const float *__restrict__ best, int k, int CB, int WB,
                                                       int DL, int64_t RBS, float *__restrict__ psum,
                                                       float *__restrict__ pcomp, int rb0,
                                                       const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    extern __shared__ float lds[];
    const int w = d + 2;
    const int P = 256 / DL;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c0 = blockIdx.y * CB;
    const int cb = min(CB, k - c0);
    const int e_lo = blockIdx.z * WB;
    const int ww = min(WB, w - e_lo);
    float *acc = lds;
    float *cmp = lds + (size_t)P * CB * WB;
    int *list = (int *)(cmp + (size_t)P * CB * WB);
    int *wcount = list + 256;
    for (int e = tid; e < P * CB * WB; e += 256) { acc[e] = 0.0f; cmp[e] = 0.0f; }
    const int64_t r_begin = (int64_t)blockIdx.x * RBS;
    const int64_t r_end = min(n, r_begin + RBS);
    const int slot = tid / DL, le = tid % DL;
    __syncthreads();
    for (int64_t r0 = r_begin; r0 < r_end; r0 += 256) {
        const int64_t r = r0 + tid;
        bool m = false;
        if (r < r_end) {
            const uint32_t L = labels[r];
            m = (L >= (uint32_t)c0) && (L < (uint32_t)(c0 + cb));
        }
        const uint64_t bal = __ballot(m);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) wcount[wave] = __popcll(bal);
        __syncthreads();
        int off = 0;
        for (int v = 0; v < wave; v++) off += wcount[v];
        const int M = wcount[0] + wcount[1] + wcount[2] + wcount[3];
        if (m) list[off + before] = tid;
        __syncthreads();
        for (int q = slot; q < M; q += P) {
            const int64_t row = r0 + list[q];
            const int L = (int)labels[row] - c0;
            float *a = acc + ((size_t)slot * CB + L) * WB;
            float *cc = cmp + ((size_t)slot * CB + L) * WB;
            for (int e = le; e < ww; e += DL) {
                const int col = e_lo + e;
                const float v = col >= 2 ? X[row * d + (col - 2)] : (col == 0 ? 1.0f : best[row]);
                neumaier(a[e], cc[e], v);
            }
        }
        __syncthreads();
    }
    const int64_t kw = (int64_t)k * w;
    for (int e = tid; e < cb * ww; e += 256) {
        const int cl = e / ww, col = e % ww;
        const size_t o = (size_t)cl * WB + col;
        float s = acc[o], c = cmp[o];
        for (int p = 1; p < P; p++) {
            neumaier(s, c, acc[(size_t)p * CB * WB + o]);
            c += cmp[(size_t)p * CB * WB + o];
        }
        const int64_t dst = (int64_t)(rb0 + blockIdx.x) * kw + (int64_t)(c0 + cl) * w + e_lo + col;
        psum[dst] = s;
        pcomp[dst] = c;
    }
}

hipError_t km_launch_accum_generic(const km_accum_plan &pl, const float *X, int64_t n, int d,
                                   const uint32_t *labels, const float *best, int k, float *psum,
                                   float *pcomp, int rb0, const int32_t *stop, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    const int dl = next_pow2(pl.wb < 256 ? pl.wb : 256);
    dim3 grid(pl.nrb, pl.ncb, pl.nwb), block(256);
    hipLaunchKernelGGL(k_accum_generic, grid, block, pl.lds, s, X, n, d, labels, best, k, pl.cb, pl.wb, dl,
                       pl.rbs, psum, pcomp, rb0, stop);
    return hipGetLastError();
}

// ------------------------------------------------------------------ partials -> totals -> update
//
// Two or three kernels finish a pass, all in a fixed order, none communicating across blocks. k_reduce_split
// cuts the row-block partials into S contiguous ranges (S depends only on the number of row-blocks and the
// entry count) and sums each range per entry in float64: sixteen waves take sixteen fixed sub-ranges and add
// their sums in wave order. The finish adds the S range sums in order into the float64 totals (columns
// [count, best, x...]) and, when the pass updates, writes the new centres float(sum / count)
// (core.py:2238-2242) into the other centre buffer, renormalised for spherical k-means (estimator.py:127-130),
// then the pass statistics in a fixed order - counts, inertia, empty clusters, the largest cluster - and the
// stopping rule (core.py:2222-2242, estimator.py:147-149); clusters that stayed empty with no row to take get
// the largest cluster's centre. Up to KM_FIN1_MAX entries one 1024-thread block does all of it (k_finish1);
// beyond, one block per cluster (k_finish) and one block for the statistics (k_stats).

static constexpr int KM_FIN1_MAX = 4096;   // entries k * (d + 2) finished by a single block (LDS)
static constexpr int KM_FIN1_SPLITS = 8;   // range sums read per entry by the single block

int km_reduce_splits(int nrb, int64_t kw, int cus) {
    int cap = kw <= KM_FIN1_MAX ? KM_FIN1_SPLITS : 64;
    // one 1024-thread block per CU at a time: keep the grid (entries / 64 x splits) within one round of blocks
    const int64_t cols = (kw + 63) / 64;
    if (kw <= KM_FIN1_MAX && cols * cap > cus) cap = (int)std::max<int64_t>(1, cus / cols);
    // with the single-block finish, about 256 partials per split (16 loads per thread of each block's sixteen
    // sub-ranges): 10M x 32, k = 64 (512 partials) 17.1 us per reduce-and-finish at 8 splits, 13.3 at 2, 14.7 at
    // 1; 100k x 32 (391 partials) 17.1 at 8, 13.2 at 2; 10M x 8 (over 3000 partials of 80 entries) 13.3 at 8,
    // 20.1 at 2
    int s = kw <= KM_FIN1_MAX ? (nrb + 255) / 256 : nrb / 16;
    if (s > cap) s = cap;
    if (s < 1) s = 1;
    return s;
}

// Block (x, y) of 1024 threads: entries 64 x .. 64 x + 63, range y of the S ranges of row-blocks. COHERENT: the range
// sums are written with device-scope stores (through to the point of coherence, no L2-wide write-back).
// With pmask, a row-block's entries of the clusters its mask leaves clear are zeros it did not write (their memory
// holds whatever an earlier pass left): each is read with the others, so the loads stay batched, and replaced by
// +0.0, which leaves the sum as it was (it starts at +0.0 and never becomes -0.0) - the same bits as without the
// mask.
template <bool COHERENT>
__device__ void reduce_split_body(const float *__restrict__ psum, const float *__restrict__ pcomp, int nrb, int64_t kw,
                                  int S, double *__restrict__ tmp, double (*part)[64], const uint32_t *__restrict__ pmask,
                                  int wd) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t e = (int64_t)blockIdx.x * 64 + lane;
    const int sp = blockIdx.y;
    const int r0 = (int)((int64_t)nrb * sp / S), r1 = (int)((int64_t)nrb * (sp + 1) / S);
    const int len = r1 - r0;
    const int q0 = r0 + (int)((int64_t)len * wave / 16), q1 = r0 + (int)((int64_t)len * (wave + 1) / 16);
    double acc = 0.0;
    if (e < kw) {
        if (!pmask) {
#pragma unroll 4
            for (int r = q0; r < q1; r++) acc += (double)psum[(int64_t)r * kw + e] + (double)pcomp[(int64_t)r * kw + e];
        } else {
            const int c = (int)(e / wd);   // the entry's cluster (wd = d + 2 entries per cluster)
            const int word = c >> 5;
            const uint32_t bit = 1u << (c & 31);
#pragma unroll 4
            for (int r = q0; r < q1; r++) {
                const double v = (double)psum[(int64_t)r * kw + e] + (double)pcomp[(int64_t)r * kw + e];
                acc += (pmask[(int64_t)r * KM_PMASK_WORDS + word] & bit) ? v : 0.0;
            }
        }
    }
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && e < kw) {
        double t = part[0][lane];
        for (int w = 1; w < 16; w++) t += part[w][lane];
        if (COHERENT) __hip_atomic_store(&tmp[(int64_t)sp * kw + e], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else tmp[(int64_t)sp * kw + e] = t;
    }
}

__global__ __launch_bounds__(1024) void k_reduce_split(const float *__restrict__ psum,
                                                       const float *__restrict__ pcomp, int nrb, int64_t kw, int S,
                                                       double *__restrict__ tmp, const int32_t *__restrict__ stop,
                                                       const uint32_t *__restrict__ pmask, int w) {
    if (stop && *stop) return;
    __shared__ double part[16][64];
    reduce_split_body<false>(psum, pcomp, nrb, kw, S, tmp, part, pmask, w);
}

hipError_t km_launch_reduce_split(const float *psum, const float *pcomp, int nrb, int64_t kw, int S, double *tmp,
                                  const int32_t *stop, hipStream_t s, const uint32_t *pmask, int w) {
    if (pmask && (w < 1 || kw % w != 0 || kw / w > 32 * KM_PMASK_WORDS)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_reduce_split, dim3((unsigned)((kw + 63) / 64), S), dim3(1024), 0, s, psum, pcomp, nrb, kw,
                       S, tmp, stop, pmask, w);
    return hipGetLastError();
}

// The pass statistics from the totals (counts in column 0, best sums in column 1), by `nthreads` threads of
// one block: strided per-thread sums over clusters ascending, then a fixed tree. Writes the control block and
// gives still-empty clusters (when no relocation is due) the largest cluster's centre.
// (count, index) pairs: the larger count wins, the smaller index on a tie
__device__ inline void max_pair(long long &mx, int &arg, long long mo, int ao) {
    if (mo > mx || (mo == mx && ao < arg)) {
        mx = mo;
        arg = ao;
    }
}

// Statistics of a pass from its totals: inertia, empty clusters, the largest cluster (first on a tie), and the
// stop flags. Each thread folds a strided set of clusters, each wave folds its lanes with a butterfly (every lane
// ends with the same bits: each step adds the same two values), and wave 0 folds the waves: two barriers.
template <int NT>
__device__ void pass_stats(const double *tot, int k, int d, float *Cnext, km_control *ctl, int pass, double tol) {
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, W = d + 2, lane = tid & 63, wave = tid >> 6;
    __shared__ double s_in[NW];
    __shared__ int s_empty[NW];
    __shared__ long long s_max[NW];
    __shared__ int s_arg[NW];
    __shared__ int s_res[2];
    double in = 0.0;
    int empty = 0;
    long long mx = -1;
    int arg = 0;
    for (int cc = tid; cc < k; cc += NT) {
        const long long n_c = llrint(tot[(int64_t)cc * W]);
        in += tot[(int64_t)cc * W + 1];
        empty += n_c == 0;
        max_pair(mx, arg, n_c, cc);
    }
    for (int off = 32; off > 0; off >>= 1) {
        in += __shfl_xor(in, off);
        empty += __shfl_xor(empty, off);
        max_pair(mx, arg, __shfl_xor(mx, off), __shfl_xor(arg, off));
    }
    if (lane == 0) {
        s_in[wave] = in;
        s_empty[wave] = empty;
        s_max[wave] = mx;
        s_arg[wave] = arg;
    }
    __syncthreads();
    if (wave == 0) {
        in = lane < NW ? s_in[lane] : 0.0;
        empty = lane < NW ? s_empty[lane] : 0;
        mx = lane < NW ? s_max[lane] : -1;
        arg = lane < NW ? s_arg[lane] : 0;
        for (int off = NW / 2; off > 0; off >>= 1) {
            in += __shfl_xor(in, off);
            empty += __shfl_xor(empty, off);
            max_pair(mx, arg, __shfl_xor(mx, off), __shfl_xor(arg, off));
        }
        if (lane == 0) {
            const double inertia = in;
            const int need_reloc = (empty > 0 && inertia > 0.0) ? 1 : 0;
            int done = 0;
            if (pass > 0 && fabs(ctl->prev - inertia) <= tol * ctl->prev) done = 1;
            ctl->prev = inertia;
            ctl->inertia = inertia;
            ctl->n_empty = empty;
            ctl->big = arg;
            ctl->need_reloc = need_reloc;
            ctl->done = done;
            ctl->iter = pass + 1;
            // a non-finite inertia (NaN or overflowing data) ends the loop at once: the caller explains it
            ctl->stop = (done || need_reloc || !isfinite(inertia)) ? 1 : 0;
            s_res[0] = (empty > 0 && !need_reloc) ? 1 : 0;
            s_res[1] = arg;
        }
    }
    __syncthreads();
    if (s_res[0]) {   // empty clusters with zero inertia: they take the largest cluster's centre
        const int big = s_res[1];
        for (int cc = 0; cc < k; cc++) {
            if (llrint(tot[(int64_t)cc * W]) != 0) continue;
            for (int j = tid; j < d; j += NT) Cnext[(int64_t)cc * d + j] = Cnext[(int64_t)big * d + j];
        }
    }
}

// Renormalise centre c of Cnext with one wave (lanes over dims, float64 sum, fixed butterfly).
__device__ void normalise_row(float *Cnext, int c, int d, int lane) {
    float *row = Cnext + (int64_t)c * d;
    double sq = 0.0;
    for (int j = lane; j < d; j += 64) sq += (double)row[j] * (double)row[j];
    for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
    const float nrm = (float)sqrt(sq);
    if (nrm > 0.0f)
        for (int j = lane; j < d; j += 64) row[j] = row[j] / nrm;
}

// The single-block finish (1024 threads; Ts: k (d + 2) doubles of LDS): range sums -> totals, the update and the
// pass statistics. COHERENT: the range sums are read with device-scope loads (written by other blocks of the same
// launch).
template <bool COHERENT>
__device__ void finish1_body(const double *__restrict__ tmp, int S, int k, int d, double *__restrict__ tot,
                             float *__restrict__ Cnext, km_control *__restrict__ ctl, int pass, double tol, int flags,
                             double *Ts) {
    const int tid = threadIdx.x, W = d + 2;
    const int kw = k * W;
    constexpr int PER = KM_FIN1_MAX / 1024;   // entries per thread
    // every load first (one round of memory latency), then the fixed-order sums
    double v[PER][KM_FIN1_SPLITS], prev[PER];
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = tid + 1024 * i;
#pragma unroll
        for (int sp = 0; sp < KM_FIN1_SPLITS; sp++) {
            double *src = const_cast<double *>(tmp) + (int64_t)sp * kw + e;
            v[i][sp] = (e < kw && sp < S)
                           ? (COHERENT ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *src)
                           : 0.0;
        }
        prev[i] = (e < kw && (flags & KM_FIN_DELTA)) ? tot[e] : 0.0;
    }
#pragma unroll
    for (int i = 0; i < PER; i++) {
        const int e = tid + 1024 * i;
        if (e >= kw) continue;
        double t = v[i][0];
#pragma unroll
        for (int sp = 1; sp < KM_FIN1_SPLITS; sp++)
            if (sp < S) t += v[i][sp];
        if ((flags & KM_FIN_DELTA) && e % W != 1) t = prev[i] + t;   // the previous totals plus their change
        Ts[e] = t;
        tot[e] = t;
    }
    __syncthreads();
    if (!(flags & KM_FIN_UPDATE)) return;
    for (int e = tid; e < k * d; e += 1024) {
        const int c = e / d, j = e - (e / d) * d;
        const long long cnt = llrint(Ts[c * W]);
        if (cnt > 0) Cnext[e] = (float)(Ts[c * W + 2 + j] / (double)cnt);
    }
    __syncthreads();
    if (flags & KM_FIN_SPHERICAL) {
        const int wave = tid >> 6, lane = tid & 63;
        for (int c = wave; c < k; c += 16)
            if (llrint(Ts[c * W]) > 0) normalise_row(Cnext, c, d, lane);
        __syncthreads();
    }
    pass_stats<1024>(Ts, k, d, Cnext, ctl, pass, tol);
}

__global__ __launch_bounds__(1024) void k_finish1(const double *__restrict__ tmp, int S, int k, int d,
                                                  double *__restrict__ tot, float *__restrict__ Cnext,
                                                  km_control *__restrict__ ctl, int pass, double tol, int flags,
                                                  const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    extern __shared__ double Ts[];   // the totals, k * (d + 2)
    finish1_body<false>(tmp, S, k, d, tot, Cnext, ctl, pass, tol, flags, Ts);
}

// k_reduce_split whose last block to finish runs the single-block finish: one launch per pass instead of two. Each
// block writes its range sums (agent-scope stores, written through to the point of coherence) and waits for them
// to complete; a block barrier orders every thread's stores before thread 0's ticket, an agent-scope release
// read-modify-write, which publishes the block's sums. The block that takes the last ticket follows it with an
// agent-scope acquire fence: its read-modify-write read the value every earlier release's sequence wrote (the
// ticket's modification order is a release sequence), so the fence synchronises with every block's release. Only
// that block's thread 0 pays for the acquire (a cache invalidation; one per block, as an acquire-release ticket
// would have it, measured 1.5-2 us slower per pass). Its barrier passes the result on to its other threads (the
// caches thread 0 invalidated are the block's); it reads the sums back with agent-scope loads (across XCDs),
// finishes, and resets the ticket for the next launch (the kernel boundary orders that store before the next
// launch's tickets).
__global__ __launch_bounds__(1024) void k_reduce_finish(const float *__restrict__ psum,
                                                        const float *__restrict__ pcomp, int nrb, int64_t kw, int S,
                                                        double *__restrict__ tmp, int k, int d,
                                                        double *__restrict__ tot, float *__restrict__ Cnext,
                                                        km_control *__restrict__ ctl, int pass, double tol, int flags,
                                                        const int32_t *__restrict__ stop,
                                                        const uint32_t *__restrict__ pmask) {
    if (stop && *stop) return;
    __shared__ double part[16][64];
    __shared__ int s_last;
    extern __shared__ double Ts[];   // the totals, k * (d + 2) (used by the last block)
    reduce_split_body<true>(psum, pcomp, nrb, kw, S, tmp, part, pmask, d + 2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned prev = __hip_atomic_fetch_add(&ctl->ticket, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == total - 1;
        if (s_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");   // every block's release, through the ticket
    }
    __syncthreads();
    if (!s_last) return;
    finish1_body<true>(tmp, S, k, d, tot, Cnext, ctl, pass, tol, flags, Ts);
    if (threadIdx.x == 0) __hip_atomic_store(&ctl->ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ __launch_bounds__(256) void k_finish(const double *__restrict__ tmp, int S, int k, int d,
                                                double *__restrict__ tot, float *__restrict__ Cnext, int flags,
                                                const float *__restrict__ Cin, const double *__restrict__ muT,
                                                const int32_t *__restrict__ dsel, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    __shared__ double red[256];
    if (dsel && *dsel == 0) {   // the pass chose its change-only sums: one range, added to the previous totals
        S = 1;
        flags |= KM_FIN_DELTA | KM_FIN_CENTRED;
    }
    const int c = blockIdx.x, W = d + 2;
    const int64_t kw = (int64_t)k * W;
    // entry j of this cluster = its S range sums added in ascending order by thread j (and every thread adds the
    // count's own, the same way, to divide by it)
    const double *src = tmp + (int64_t)c * W;
    const bool delta = (flags & KM_FIN_DELTA) != 0;
    double cntd = 0.0;
    for (int sp = 0; sp < S; sp++) cntd += src[(int64_t)sp * kw];
    if (delta) cntd = tot[(int64_t)c * W] + cntd;
    const long long cnt = llrint(cntd);
    const bool update = (flags & KM_FIN_UPDATE) != 0;
    __syncthreads();   // every thread has read the previous count before thread 0 overwrites it
    const bool centred = (flags & KM_FIN_CENTRED) != 0;
    double u = 0.0;   // this thread's part of the cluster's centred inertia term
    for (int j = threadIdx.x; j < W; j += 256) {
        double v = 0.0;
        for (int sp = 0; sp < S; sp++) v += src[(int64_t)sp * kw + j];
        if (delta && j != 1) v = tot[(int64_t)c * W + j] + v;   // the previous totals plus their change
        tot[(int64_t)c * W + j] = v;
        if (update && j >= 2 && cnt > 0) Cnext[(int64_t)c * d + (j - 2)] = (float)(v / (double)cnt);
        if (centred && j >= 2) {   // n |D|^2 - 2 D . (S - n mu), D = c - mu, for this dim
            const double m = muT[j - 2], D = (double)Cin[(int64_t)c * d + (j - 2)] - m;
            u += (double)cnt * D * D - 2.0 * D * (v - (double)cnt * m);
        }
    }
    if (centred) {   // the cluster's inertia from the totals (the pass read no row distances): T + sum_c u_c
        red[threadIdx.x] = u;
        __syncthreads();
        for (int h = 128; h > 0; h >>= 1) {
            if (threadIdx.x < h) red[threadIdx.x] += red[threadIdx.x + h];
            __syncthreads();
        }
        if (threadIdx.x == 0) tot[(int64_t)c * W + 1] = red[0] + (c == 0 ? muT[d] : 0.0);
    }
    if (update && (flags & KM_FIN_SPHERICAL) && cnt > 0) {
        __syncthreads();
        if (threadIdx.x < 64) normalise_row(Cnext, c, d, threadIdx.x);
    }
}

__global__ __launch_bounds__(256) void k_stats(const double *__restrict__ tot, int k, int d,
                                               float *__restrict__ Cnext, km_control *__restrict__ ctl, int pass,
                                               double tol, const int32_t *__restrict__ stop) {
    if (stop && *stop) return;
    pass_stats<256>(tot, k, d, Cnext, ctl, pass, tol);
}

hipError_t km_launch_reduce_finish(const float *psum, const float *pcomp, int nrb, int64_t kw, int S, double *tmp,
                                   int k, int d, double *tot, float *Cnext, km_control *ctl, int pass, double tol,
                                   int flags, const int32_t *stop, hipStream_t s, const uint32_t *pmask) {
    if (pmask && (kw != (int64_t)k * (d + 2) || k > 32 * KM_PMASK_WORDS)) return hipErrorInvalidValue;
    if (kw <= KM_FIN1_MAX && S <= KM_FIN1_SPLITS) {
        hipLaunchKernelGGL(k_reduce_finish, dim3((unsigned)((kw + 63) / 64), S), dim3(1024), (size_t)kw * sizeof(double),
                           s, psum, pcomp, nrb, kw, S, tmp, k, d, tot, Cnext, ctl, pass, tol, flags, stop, pmask);
        return hipGetLastError();
    }
    hipError_t e = km_launch_reduce_split(psum, pcomp, nrb, kw, S, tmp, stop, s, pmask, d + 2);
    if (e != hipSuccess) return e;
    return km_launch_finish(tmp, S, k, d, tot, Cnext, ctl, pass, tol, flags, stop, s);
}

hipError_t km_launch_finish(const double *tmp, int S, int k, int d, double *tot, float *Cnext, km_control *ctl,
                            int pass, double tol, int flags, const int32_t *stop, hipStream_t s, const float *Cin,
                            const double *muT, const int32_t *dsel) {
    const int64_t kw = (int64_t)k * (d + 2);
    if (((flags & KM_FIN_CENTRED) || dsel) && (!Cin || !muT)) return hipErrorInvalidValue;
    if (kw <= KM_FIN1_MAX && S <= KM_FIN1_SPLITS && !(flags & KM_FIN_CENTRED) && !dsel) {
        hipLaunchKernelGGL(k_finish1, dim3(1), dim3(1024), (size_t)kw * sizeof(double), s, tmp, S, k, d, tot, Cnext,
                           ctl, pass, tol, flags, stop);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_finish, dim3(k), dim3(256), 0, s, tmp, S, k, d, tot, Cnext, flags, Cin, muT, dsel, stop);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !(flags & KM_FIN_UPDATE)) return e;
    hipLaunchKernelGGL(k_stats, dim3(1), dim3(256), 0, s, tot, k, d, Cnext, ctl, pass, tol, stop);
    return hipGetLastError();
}

// Spherical k-means: each centre divided by its length (float32 division by the float32-rounded norm, which is
// summed in float64), a zero centre left as is.
__global__ __launch_bounds__(64) void k_normalise(float *__restrict__ C, int k, int d) {
    const int c = blockIdx.x;
    if (c >= k) return;
    float *row = C + (size_t)c * d;
    double s = 0.0;
    for (int j = threadIdx.x; j < d; j += 64) s += (double)row[j] * (double)row[j];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    const float nrm = (float)sqrt(s);
    if (nrm > 0.0f)
        for (int j = threadIdx.x; j < d; j += 64) row[j] = row[j] / nrm;
}

hipError_t km_launch_normalise(float *C, int k, int d, hipStream_t s) {
    hipLaunchKernelGGL(k_normalise, dim3(k), dim3(64), 0, s, C, k, d);
    return hipGetLastError();
}
