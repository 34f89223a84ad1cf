// Per-cluster float64 sums over rows listed in cluster order, in fixed chunks: the last step of the wide-row
// path's accumulation (rows sorted by label) and of its change-only passes (changed rows' +/- entries sorted by
// label), and of the rows loop's above 4096 centres (core.py:934-994, 424-449: the reference's sorted
// accumulation).
//
// The counting sort leaves each cluster's positions contiguous, in row order (or entry order). Wave q takes the
// positions [q Q, (q + 1) Q), whatever clusters they belong to, so every wave has the same work however unevenly
// the rows fall among the clusters. It loads the positions' rows, labels and addresses lane-parallel, adds the
// rows in position order, several in flight, into float64 sums (lane owns dims lane, lane + 64, ...) and closes a
// piece at every change of cluster. A cluster whose positions lie inside the chunk is complete and is written to
// its totals [count, best, x]; one whose positions run past the chunk's edge leaves a piece, in the chunk's head
// slot for the cluster holding its first position, in the tail slot for the one holding its last. One block per
// cluster then adds a spanning cluster's pieces in chunk order (and writes zeros for an empty one). Every order is
// fixed, so reruns give the same bits.
//
// The best column: MODE 0 adds best[] of each row; MODE 1 adds each row's distance to its cluster's centre in FMA
// form (float32 per lane over its dims, float64 across rows, the lanes added in a fixed butterfly: the sum of the
// rows' direct-form distances to float32 rounding) for passes whose rescoring left some rows without one; MODE 2
// (change entries: +row under the new label, -row under the old, the row's slice found in the slice table) adds
// signed rows and leaves the column zero.
#include "km_internal.h"

namespace {

typedef __attribute__((address_space(1))) float gfloat;

template <int MODE>
constexpr int kc_q() { return MODE == 2 ? 64 : 256; }   // positions per wave

template <int NJ, int MODE>   // NJ: dims per lane, ceil(d / 64)
__global__ __launch_bounds__(256) void k_chunk_sums(const float *__restrict__ X, const km_slice *__restrict__ slices,
                                                    int nslices, int d,
                                                    const uint32_t *__restrict__ lab,
                                                    const uint32_t *__restrict__ erow,
                                                    const float *__restrict__ best, const float *__restrict__ C,
                                                    const uint32_t *__restrict__ perm,
                                                    const uint32_t *__restrict__ counts,
                                                    const uint32_t *__restrict__ base,
                                                    const uint32_t *__restrict__ npos_dev, int64_t npos,
                                                    double *__restrict__ pieces, double *__restrict__ tmp,
                                                    const int32_t *__restrict__ gate) {
    constexpr int Q = kc_q<MODE>();
    if (gate && *gate) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t q = (int64_t)blockIdx.x * 4 + wave;
    const int64_t E = MODE == 2 ? 2 * (int64_t)*npos_dev : npos;
    const int64_t e0 = q * Q;
    if (e0 >= E) return;   // whole waves leave; the kernel has no barriers
    const int64_t e1 = (E - e0 < Q) ? E : e0 + Q;
    const int W = d + 2;
    double acc[NJ];
#pragma unroll
    for (int i = 0; i < NJ; i++) acc[i] = 0.0;
    double cntd = 0.0, accb = 0.0;
    float cv[MODE == 1 ? NJ : 1];
    uint32_t cur = 0xffffffffu;
    auto load_centre = [&](uint32_t cl) {
        if constexpr (MODE == 1) {
            const float *cc = C + (int64_t)cl * d;
#pragma unroll
            for (int i = 0; i < NJ; i++) cv[i] = cc[min(lane + 64 * i, d - 1)];
#pragma unroll
            for (int i = 0; i < NJ; i++)
                if (lane + 64 * i >= d) cv[i] = 0.0f;
        }
    };
    auto flush = [&](uint32_t cl) {
        double col1 = 0.0;
        if constexpr (MODE == 1) {   // the lanes' partial distances, added in a fixed butterfly
            col1 = accb;
            for (int off = 32; off > 0; off >>= 1) col1 += __shfl_xor(col1, off);
        } else if constexpr (MODE == 0) {
            col1 = accb;   // the same in every lane
        }
        const int64_t b = base[cl], e = b + counts[cl];
        double *dst = (b >= e0 && e <= e1) ? tmp + (int64_t)cl * W
                                           : pieces + (q * 2 + (b <= e0 ? 0 : 1)) * (int64_t)W;
        if (lane == 0) {
            dst[0] = cntd;
            dst[1] = col1;
        }
#pragma unroll
        for (int i = 0; i < NJ; i++) {
            const int j = lane + 64 * i;
            if (j < d) dst[2 + j] = acc[i];
            acc[i] = 0.0;
        }
        cntd = 0.0;
        accb = 0.0;
    };
    for (int64_t s0 = e0; s0 < e1; s0 += 64) {
        const int ns = (int)((e1 - s0) < 64 ? (e1 - s0) : 64);
        // lane L: sorted position s0 + L - its label, its row's address, its sign, its best
        uint32_t my_lab = 0xffffffffu, my_er = 0;
        float my_best = 0.0f;
        const float *my_x = MODE == 2 ? slices[0].X : X;
        if (lane < ns) {
            const uint32_t pe = perm[s0 + lane];
            my_lab = lab[pe];
            if constexpr (MODE == 2) {
                my_er = erow[pe];
                const int64_t r = (int64_t)(my_er & 0x7fffffffu);
                int sl = 0;
                while (sl + 1 < nslices && slices[sl + 1].row0 <= r) sl++;
                my_x = slices[sl].X + (r - slices[sl].row0) * d;
            } else {
                my_x = X + (int64_t)pe * d;
                if constexpr (MODE == 0) my_best = best[pe];
            }
        }
        const uint64_t my_xa = (uint64_t)(uintptr_t)my_x;
        if (cur == 0xffffffffu) {   // the chunk's first cluster
            cur = (uint32_t)__shfl((int)my_lab, 0);
            load_centre(cur);
        }
        for (int t = 0; t < ns; t += 4) {
            // four rows' loads, unconditional (a lane past the last dim reads dim d - 1, a slot past the end reads
            // row t again), then the adds in position order, masked: a guarded load becomes a branch and a wait
            const gfloat *x[4];
#pragma unroll
            for (int u = 0; u < 4; u++)
                x[u] = (const gfloat *)(uintptr_t)(uint64_t)__shfl((long long)my_xa, t + u < ns ? t + u : t);
            float v[4][NJ];
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int i = 0; i < NJ; i++) {   // the full accumulation reads each row once: non-temporal
                    const gfloat *a = &x[u][min(lane + 64 * i, d - 1)];
                    v[u][i] = MODE == 2 ? *a : __builtin_nontemporal_load(a);
                }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                if (t + u >= ns) break;   // wave-uniform
                const uint32_t lb = (uint32_t)__shfl((int)my_lab, t + u);
                if (lb != cur) {
                    flush(cur);
                    cur = lb;
                    load_centre(cur);
                }
#pragma unroll
                for (int i = 0; i < NJ; i++)
                    if (lane + 64 * i >= d) v[u][i] = 0.0f;
                if constexpr (MODE == 2) {
                    const bool neg = ((uint32_t)__shfl((int)my_er, t + u) >> 31) != 0;
#pragma unroll
                    for (int i = 0; i < NJ; i++) acc[i] = neg ? acc[i] - (double)v[u][i] : acc[i] + (double)v[u][i];
                    cntd += neg ? -1.0 : 1.0;
                } else {
#pragma unroll
                    for (int i = 0; i < NJ; i++) acc[i] += (double)v[u][i];
                    cntd += 1.0;
                    if constexpr (MODE == 0) {
                        accb += (double)__shfl(my_best, t + u);
                    } else {
                        float ds = 0.0f;
#pragma unroll
                        for (int i = 0; i < NJ; i++) {
                            const float tt = v[u][i] - cv[i];   // 0 - 0 past the last dim
                            ds = __builtin_fmaf(tt, tt, ds);
                        }
                        accb += (double)ds;
                    }
                }
            }
        }
    }
    flush(cur);
}

// Block per cluster: zeros for an empty cluster; for one whose positions span several chunks, its pieces in
// chunk order (the head slot of every chunk whose first position it holds, the tail slot of the chunk it starts in
// otherwise); one inside a single chunk was written whole by that chunk's wave.
template <int MODE>
__global__ __launch_bounds__(256) void k_chunk_combine(const uint32_t *__restrict__ counts,
                                                       const uint32_t *__restrict__ base, int d,
                                                       const double *__restrict__ pieces, double *__restrict__ tmp,
                                                       const int32_t *__restrict__ gate) {
    constexpr int Q = kc_q<MODE>();
    if (gate && *gate) return;
    const int c = blockIdx.x, W = d + 2;
    const int64_t cnt = counts[c], b = base[c];
    double *dst = tmp + (int64_t)c * W;
    if (cnt == 0) {
        for (int j = threadIdx.x; j < W; j += 256) dst[j] = 0.0;
        return;
    }
    const int64_t q0 = b / Q, q1 = (b + cnt - 1) / Q;
    if (q0 == q1) return;
    for (int j = threadIdx.x; j < W; j += 256) {
        double t = 0.0;
        for (int64_t qa = q0; qa <= q1; qa += 8) {   // eight loads in flight, added in chunk order
            double v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int64_t qq = qa + u;
                v[u] = qq <= q1 ? pieces[(qq * 2 + (b <= qq * Q ? 0 : 1)) * (int64_t)W + j] : 0.0;
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (qa + u <= q1) t += v[u];
        }
        dst[j] = t;
    }
}

typedef void (*chunk_fn)(const float *, const km_slice *, int, int, const uint32_t *, const uint32_t *, const float *,
                         const float *, const uint32_t *, const uint32_t *, const uint32_t *, const uint32_t *, int64_t,
                         double *, double *, const int32_t *);

template <int MODE>
chunk_fn chunk_for(int nj) {
    switch (nj) {
        case 1: return k_chunk_sums<1, MODE>;
        case 2: return k_chunk_sums<2, MODE>;
        case 3: return k_chunk_sums<3, MODE>;
        case 4: return k_chunk_sums<4, MODE>;
        case 5: return k_chunk_sums<5, MODE>;
        case 6: return k_chunk_sums<6, MODE>;
        case 7: return k_chunk_sums<7, MODE>;
        case 8: return k_chunk_sums<8, MODE>;
        case 9: return k_chunk_sums<9, MODE>;
        case 10: return k_chunk_sums<10, MODE>;
        case 11: return k_chunk_sums<11, MODE>;
        case 12: return k_chunk_sums<12, MODE>;
        case 13: return k_chunk_sums<13, MODE>;
        case 14: return k_chunk_sums<14, MODE>;
        case 15: return k_chunk_sums<15, MODE>;
        case 16: return k_chunk_sums<16, MODE>;
        case 20: return k_chunk_sums<20, MODE>;
        case 24: return k_chunk_sums<24, MODE>;
        default: return nullptr;
    }
}

}  // namespace

int64_t km_chunk_piece_doubles(int64_t npos, int d, int mode) {
    const int Q = mode == 2 ? kc_q<2>() : kc_q<0>();
    return (npos + Q - 1) / Q * 2 * (int64_t)(d + 2);
}

hipError_t km_launch_chunk_sums(int mode, const float *X, const km_slice *slices, int nslices, int d, const uint32_t *lab,
                                const uint32_t *erow, const float *best, const float *C, const uint32_t *perm,
                                const uint32_t *counts, const uint32_t *base, int k, const uint32_t *npos_dev,
                                int64_t npos, double *pieces, double *tmp, const int32_t *gate, hipStream_t s) {
    if (d < 1 || d > KM_CHUNK_MAX_DIMS || npos < 1 || mode < 0 || mode > 2 || k < 1 ||
        (mode == 2 ? (!slices || nslices < 1) : !X))
        return hipErrorInvalidValue;
    // dims per lane: ceil(d / 64), above 16 rounded up to 20 or 24 (the lanes past the last dim add zeros)
    int nj = (d + 63) / 64;
    if (nj > 16) nj = nj <= 20 ? 20 : 24;
    const chunk_fn fn = mode == 0 ? chunk_for<0>(nj) : mode == 1 ? chunk_for<1>(nj) : chunk_for<2>(nj);
    if (!fn) return hipErrorInvalidValue;
    const int Q = mode == 2 ? kc_q<2>() : kc_q<0>();
    const int64_t nq = (npos + Q - 1) / Q;
    hipLaunchKernelGGL(fn, dim3((unsigned)((nq + 3) / 4)), dim3(256), 0, s, X, slices, nslices, d, lab, erow, best, C,
                       perm, counts, base, npos_dev, npos, pieces, tmp, gate);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (mode == 2)
        hipLaunchKernelGGL(k_chunk_combine<2>, dim3(k), dim3(256), 0, s, counts, base, d, pieces, tmp, gate);
    else
        hipLaunchKernelGGL(k_chunk_combine<0>, dim3(k), dim3(256), 0, s, counts, base, d, pieces, tmp, gate);
    return hipGetLastError();
}
