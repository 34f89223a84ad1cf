// Internal declarations shared by the runtime (km_api.hip) and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Device-resident state of a fit loop. One per context; the update kernels read and write it so that
// iterations can run back to back with no host round trip.
struct km_control {
    int32_t iter;        // passes completed in the current loop (the update stage of pass p sets it to p+1)
    int32_t stop;        // set when no further pass may run: converged, or an empty cluster needs relocating
    int32_t done;        // |prev - inertia| <= tol * prev held at the last completed pass
    int32_t need_reloc;  // the last completed pass left clusters empty while some row had best > 0
    int32_t n_empty;     // empty clusters in the last completed pass
    int32_t big;         // first index of the largest count in the last completed pass
    int32_t pad0, pad1;
    double inertia;      // inertia of the last completed pass (of its input centres)
    double prev;         // inertia of the pass before it
    double tol;
    uint64_t fallback_rows;  // rows the MFMA screen left to a full rescoring, summed over passes
};

// Kernel ids for timing (order fixed; names in km_kernel_names).
enum km_kernel_id {
    KK_PREP = 0,
    KK_ASSIGN_ROWS,
    KK_ACCUM_GENERIC,
    KK_REDUCE,
    KK_UPDATE_STATS,
    KK_UPDATE_CENTRES,
    KK_NORMALISE,
    KK_FUSED_ROWS,
    KK_FUSED_MFMA,
    KK_ASSIGN_MFMA,
    KK_COUNT
};
extern const char *const km_kernel_names[KK_COUNT];

// Per-pass centre-derived data for the screens.
struct km_centre_aux {
    float *csq;      // (kpad) |c|^2 rounded to float32 (+inf for padding centres)
    float *cnorm;    // (kpad) |c| rounded up
    float *maxes;    // [0] max |c|, [1] max |c|^2 over real centres
    uint16_t *cb;    // (kpad, dpad) bf16 of -2*c in the MFMA operand layout, or null
};

// ---- launchers (defined in the kernel translation units) ----
// Generic exact assignment (direct form over every centre). labels/best may be null. stop: gate or null.
hipError_t km_launch_assign_rows(const float *X, int64_t n, int d, const float *C, int k, uint32_t *labels,
                                 float *best, const int32_t *stop, hipStream_t s);

// Generic deterministic accumulation of [count, best, x] into per-row-block partials.
struct km_accum_plan {
    int64_t rbs;     // rows per row-block
    int nrb;         // row-blocks
    int cb, ncb;     // clusters per cluster-block, cluster-blocks
    int wb, nwb;     // columns per column-block, column-blocks
    size_t lds;      // dynamic LDS bytes
};
km_accum_plan km_plan_accum_generic(int64_t n, int d, int k);
hipError_t km_launch_accum_generic(const km_accum_plan &pl, const float *X, int64_t n, int d,
                                   const uint32_t *labels, const float *best, int k, float *psum,
                                   float *pcomp, int rb0, const int32_t *stop, hipStream_t s);

// Partials (nrb, k*w) sum+comp -> totals (k*w) float64 in a fixed order; tmp holds km_reduce_tmp_doubles.
size_t km_reduce_tmp_doubles(int nrb, int64_t kw);
hipError_t km_launch_reduce(const float *psum, const float *pcomp, int nrb, int64_t kw, double *tmp, double *tot,
                            const int32_t *stop, hipStream_t s);

// Update stage. stats: counts, inertia, empties, argmax, tol test; centres: C <- sums / counts.
hipError_t km_launch_update_stats(const double *tot, int k, int w, km_control *ctl, int pass, double tol,
                                  hipStream_t s);
hipError_t km_launch_update_centres(const double *tot, int k, int d, km_control *ctl, int pass, float *C,
                                    hipStream_t s);
hipError_t km_launch_normalise(float *C, int k, int d, const km_control *ctl, int pass, hipStream_t s);

// Centre-derived data for the MFMA screen; also zero-fills nothing. kpad/dpad: padded sizes.
hipError_t km_launch_prep(const float *C, int k, int d, int kpad, int dpad, km_centre_aux aux,
                          const int32_t *stop, hipStream_t s);

// MFMA-screened exact assignment. Fused variant also accumulates into partials (one row-block per block).
struct km_mfma_plan {
    int ok;          // 0 if the shape is not served
    int kpad, dpad;  // padded centre count and dims
    int64_t rbs;     // rows per block (fused)
    int nrb;         // blocks
    int waves;       // waves per block
    size_t lds;
};
km_mfma_plan km_plan_mfma(int64_t n, int d, int k, int fused);
hipError_t km_launch_mfma(const km_mfma_plan &pl, int fused, const float *X, int64_t n, int d, const float *C,
                          int k, km_centre_aux aux, uint32_t *labels, float *best, float *psum, float *pcomp,
                          int rb0, km_control *ctl, const int32_t *stop, hipStream_t s);

// Fused single-read pass for dims <= 16: exact rows loop + deterministic accumulation into per-block partials.
struct km_lowd_plan {
    int ok;          // 0 if the shape is not served (dims > 16, LDS too small, misaligned rows)
    int64_t rbs;     // rows per block
    int nrb;         // blocks
    size_t lds;      // dynamic LDS bytes
};
km_lowd_plan km_plan_lowd(int64_t n, int d, int k, bool aligned);
hipError_t km_launch_lowd(const km_lowd_plan &pl, const float *X, int64_t n, int d, const float *C, int k,
                          uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, const int32_t *stop,
                          hipStream_t s);
