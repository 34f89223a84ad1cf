// Internal declarations shared by the runtime (km_api.hip) and the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((address_space(3))) void *lds_vptr;
typedef __attribute__((address_space(1))) void *gbl_vptr;

// Direct global->LDS load of 16 bytes per lane (global_load_lds_dwordx4: lane i's bytes land at dst + 16 i). It is
// issued from inline assembly so that the compiler neither tracks it nor waits for it: the caller's own
// s_waitcnt vmcnt(n) says when the data is in LDS. (Through the builtin, the compiler may wait for every pending
// direct load before the next LDS access of any kind: in the fused kernel's loop it did, before the first read of
// the current block, which drained the double buffer at every step.) M0 holds the
// wave-uniform LDS address and needs one wait state before the load reads it. M0 is a register the compiler
// reserves (it sets it before each of its own uses), so naming it as clobbered is harmless and only warned about.
// NT: the non-temporal hint, for data a pass reads once (the rows, the per-row label state): on MI355X a plain
// streaming read reaches 7.0-7.1 TB/s with it and 6.2-6.3 without.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
template <bool NT = false>
__device__ __forceinline__ void lds_dma16(const void *src, lds_vptr dst) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
    if constexpr (NT)
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "s"(m) : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m) : "memory", "m0");
}
#pragma clang diagnostic pop

// Device-resident state of a fit loop. One per context; the update kernels read and write it so that
// iterations can run back to back with no host round trip.
struct km_control {
    int32_t iter;        // passes completed in the current loop (the update stage of pass p sets it to p+1)
    int32_t stop;        // set when no further pass may run: converged, an empty cluster needs relocating, or
                         // the inertia came out non-finite
    int32_t done;        // |prev - inertia| <= tol * prev held at the last completed pass
    int32_t need_reloc;  // the last completed pass left clusters empty while some row had best > 0
    int32_t n_empty;     // empty clusters in the last completed pass
    int32_t big;         // first index of the largest count in the last completed pass
    uint32_t n_over;     // rows the wide-row screen listed for a full scan in the running pass
    uint32_t n_multi;    // rows the wide-row screen listed with two or more candidates in the running pass
    double inertia;      // inertia of the last completed pass (of its input centres)
    double prev;         // inertia of the pass before it
    double tol;
    uint64_t fallback_rows;  // rows the MFMA screen left to a full rescoring, summed over passes
    uint32_t ticket;         // blocks of the running reduce that have written their range sums (reset by the last)
    uint32_t pad_;
};

// What the planners need to know of the device a context runs on (read once, in km_create).
struct km_device_info {
    int cus;          // compute units
    size_t lds_max;   // LDS bytes one workgroup may use
};

// Kernel ids for timing (order fixed; names in km_kernel_names).
enum km_kernel_id {
    KK_ASSIGN_ROWS = 0,
    KK_ACCUM_GENERIC,
    KK_REDUCE,
    KK_FINISH,
    KK_NORMALISE,
    KK_FUSED_LOWD,
    KK_FUSED_MFMA,
    KK_BIG_PREP,
    KK_BIG_SCREEN,
    KK_BIG_RESCORE,
    KK_BIG_ACCUM,
    KK_SEED_PP,
    KK_RELOCATE,
    KK_CHANGE,   // the wide-row fit loop's change count, gate and change-only sums
    KK_BOUNDS,   // the per-centre bounds: drift, sample count, decision
    KK_BOUNDS_LIST,   // the per-centre bounds: a pass's candidate lists
    KK_BIG_SCREEN_BND,   // the screen of a pass that builds the per-centre bounds
    KK_BOUNDS_SAMPLE,    // the per-centre bounds' sample tiles: count and fresh bounds
    KK_COUNT
};
extern const char *const km_kernel_names[KK_COUNT];

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
// max_rb > 0: at most that many row-blocks (longer blocks), so the partials fit a caller's budget
km_accum_plan km_plan_accum_generic(int64_t n, int d, int k, int64_t max_rb = 0);
hipError_t km_launch_accum_generic(const km_accum_plan &pl, const float *X, int64_t n, int d,
                                   const uint32_t *labels, const float *best, int k, float *psum,
                                   float *pcomp, int rb0, const int32_t *stop, hipStream_t s);

// Partials (nrb, k*w) sum+comp -> float64 sums of S = km_reduce_splits(nrb, k*w) fixed ranges: tmp (S, k*w).
// pmask (optional, KM_PMASK_WORDS words per row-block): bit c set where the block wrote cluster c's row of
// partials; a clear bit means that row is all zeros and was not written, and the reduce skips it (w = d + 2
// entries per cluster row).
#define KM_PMASK_WORDS 4
int km_reduce_splits(int nrb, int64_t kw, int cus);
hipError_t km_launch_reduce_split(const float *psum, const float *pcomp, int nrb, int64_t kw, int S, double *tmp,
                                  const int32_t *stop, hipStream_t s, const uint32_t *pmask = nullptr, int w = 1);

// Range sums -> totals (k, d+2). With KM_FIN_UPDATE also the new centres into Cnext and the pass statistics and
// stopping rule into ctl (pass `pass`, tolerance tol); KM_FIN_SPHERICAL renormalises the new centres.
#define KM_FIN_UPDATE 1
#define KM_FIN_SPHERICAL 2
#define KM_FIN_DELTA 4    // the range sums are the change since the previous pass: added to tot (the inertia
                          // column, column 1, is the pass's own)
#define KM_FIN_CENTRED 8  // column 1 from the totals: T + sum_c (n_c |c - mu|^2 - 2 (c - mu).(S_c - n_c mu)), with
                          // the pass's centres Cin and muT = [mu (d), T] (the multi-block finish)
hipError_t km_launch_finish(const double *tmp, int S, int k, int d, double *tot, float *Cnext, km_control *ctl,
                            int pass, double tol, int flags, const int32_t *stop, hipStream_t s,
                            const float *Cin = nullptr, const double *muT = nullptr,
                            const int32_t *dsel = nullptr);
// dsel (a gate word of the change-only accumulation): when it reads 0 the finish takes S = 1 change-only range and
// adds KM_FIN_DELTA | KM_FIN_CENTRED to flags
// ---- change-only accumulation of the wide-row fit loop (km_wdelta.hip)
struct km_slice {
    const float *X;   // the slice's rows
    int64_t row0;     // its first row in the data set
};
int64_t km_wd_blocks(int64_t n);        // count blocks: bcnt takes km_wd_blocks(n) + 1 words
int64_t km_wd_stat_blocks(int64_t n);   // mean / scatter blocks of one slice
int km_wd_max_dims();
// mu (d float64) and T = sum |x - mu|^2 into mu_T[0 .. d]; part: the slices' km_wd_stat_blocks x (d + 1) doubles
hipError_t km_launch_wd_stats(const km_slice *slices_h, const int64_t *rows, int nslices, int d, double *part,
                              double *mu_T, hipStream_t s);
// The changed rows of this pass (lab vs prev over all n rows) and the gate words gate[0] (nonzero: no change-only
// sums this pass) and gate[1] (nonzero: no full accumulation): change-only when at most `limit` rows changed
hipError_t km_launch_wd_gate(const uint32_t *lab, const uint32_t *prev, int64_t n, int64_t limit, uint32_t *bcnt,
                             int32_t *gate, const int32_t *stop, hipStream_t s);
// The change sums into tmp (k (d + 2), column 1 zero) when gate[0] is 0. elab, erow and perm hold 2 limit words
// each, H km_sorted_blocks(2 limit) x k counters, counts / base k words, pieces km_chunk_piece_doubles(2 limit, d,
// 2); slices_d a device copy of the slice table
hipError_t km_launch_wd_accum(const km_slice *slices_d, int nslices, int64_t n, int d, const uint32_t *lab,
                              const uint32_t *prev, int k, int64_t limit, const uint32_t *bcnt, uint32_t *elab,
                              uint32_t *erow, uint32_t *H, uint32_t *counts, uint32_t *base, uint32_t *perm,
                              double *pieces, double *tmp, const int32_t *gate, hipStream_t s);
hipError_t km_launch_normalise(float *C, int k, int d, hipStream_t s);
// Streaming read of `bytes` (a multiple of 16) at x by `blocks` blocks of 256 threads; out holds blocks * 256 floats.
hipError_t km_launch_stream_read(const void *x, int64_t bytes, float *out, int blocks, hipStream_t s);
// The reduce and the finish in one launch where the single-block finish serves the shape (the reduce's last block
// finishes), else the two launches.
hipError_t km_launch_reduce_finish(const float *psum, const float *pcomp, int nrb, int64_t kw, int S, double *tmp,
                                   int k, int d, double *tot, float *Cnext, km_control *ctl, int pass, double tol,
                                   int flags, const int32_t *stop, hipStream_t s, const uint32_t *pmask = nullptr);

// Greedy k-means++ on a device-resident sample of the rows, held transposed as ST (d x m) and row-major as SR
// (m x d) (km_seed.hip). km_pp_trials(k) candidates per round (at most KM_PP_MAX_TRIALS); ws:
// km_pp_workspace(m, k) bytes; seeds_h: host, k - 1 round seeds; C: the k picked rows (device).
#define KM_PP_MAX_TRIALS 16
int km_pp_trials(int k);
size_t km_pp_workspace(int64_t m, int k);
hipError_t km_launch_pp_gather(const float *X, const int64_t *idx, int64_t j0, int64_t j1, int64_t m, int d,
                               float *ST, float *SR, hipStream_t s);
hipError_t km_launch_pp(const float *ST, const float *SR, int64_t m, int d, int k, int64_t first,
                        const uint64_t *seeds_h, void *ws, float *C, hipStream_t s);

// MFMA-screened exact assignment. Fused variant also accumulates into partials (one per workgroup, which takes
// blocks of 64 rows per wave round-robin).
struct km_mfma_plan {
    int ok;          // 0 if the shape is not served
    int kpad, dpad;  // padded centre count and dims
    int64_t rbs;     // at most this many rows per workgroup (fused)
    int nrb;         // blocks
    int waves;       // waves per block
    size_t lds;
};
// max_blocks > 0: at most that many workgroups (each takes more row blocks), so the partials fit a budget
km_mfma_plan km_plan_mfma(const km_device_info &dev, int64_t n, int d, int k, int64_t max_blocks = 0);
// want_best: every row's exact direct-form distance (labels/best outputs); without it, rows the screen settles
// alone add an FMA-form distance to the pass inertia (their labels are exact either way).
// Label state of a fit (lmode, without want_best): 0 none; KM_LSTATE_RECORD every row's label goes to lout (one
// byte per row, the pass accumulates every row); KM_LSTATE_DELTA the pass reads the previous labels from lprev
// (buffer padded by 64 bytes), accumulates only the rows whose label changed (+1, +x to the new cluster; -1, -x
// to the old), so its partials hold the change of the totals, and writes the changed labels to lout.
#define KM_LSTATE_NONE 0
#define KM_LSTATE_RECORD 1
#define KM_LSTATE_DELTA 2
// scan_only (KM_LSTATE_DELTA passes): the kernel without the candidate lists for waves with many open rows, every
// open row scanned by the whole wave (smaller; for data whose open rows are rare). pmask (KM_LSTATE_DELTA passes,
// optional): each block writes only the rows of partials of the clusters its changed rows left or joined (and
// cluster 0's, which carries the inertia), and marks them in its KM_PMASK_WORDS words at pmask[(rb0 + block) *
// KM_PMASK_WORDS]; the reduce must then be given the same pmask.
hipError_t km_launch_mfma(const km_mfma_plan &pl, int want_best, const float *X, int64_t n, int d, const float *C,
                          int k, uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, km_control *ctl,
                          const uint8_t *lprev, uint8_t *lout, int lmode, const int32_t *stop, hipStream_t s,
                          int scan_only = 0, uint32_t *pmask = nullptr);

// Fused single-read pass for dims <= 16: exact rows loop + deterministic accumulation into per-block partials.
struct km_lowd_plan {
    int ok;          // 0 if the shape is not served (dims > 16, LDS too small, misaligned rows)
    int screen;      // 1: float32 expanded-form screen + window, direct form on the winner only
    int64_t rbs;     // rows per block
    int nrb;         // blocks
    size_t lds;      // dynamic LDS bytes
    int lsh;         // the wave keeps 64 >> lsh tile columns; 1 << lsh lanes take turns on each
};
km_lowd_plan km_plan_lowd(const km_device_info &dev, int64_t n, int d, int k, bool aligned, int64_t max_blocks = 0);
hipError_t km_launch_lowd(const km_lowd_plan &pl, const float *X, int64_t n, int d, const float *C, int k,
                          uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, const int32_t *stop,
                          hipStream_t s);

// Wide rows (16 < dims <= KM_BIG_MAX_DIMS, k <= KM_BIG_MAX_K): bf16 MFMA screen keeping up to 16 keys per half-row
// (32 above 768 dims), exact rescoring of the candidates, stable counting sort by label and per-cluster float64
// sums.
struct km_big_plan {
    int ok;
    int DS;          // MFMA K-steps over the padded dims (16 DS >= dims)
    int kpad;        // centres padded to a multiple of 32
    int nchunks;     // kpad / 32
    int ib;          // centre-index bits packed into keys (0: keys carry no index, k > KM_BIG_PACK_MAX_K)
    int64_t ntiles;  // 32-row tiles
    int nb;          // 4096-row blocks of the sort
};
// Largest k whose keys carry the centre index in their low mantissa bits (12 bits: a relative perturbation of
// 2^-11 at most); above it, up to KM_BIG_MAX_K, the screen keeps each listed key's index beside it.
#define KM_BIG_PACK_MAX_K 4096
#define KM_BIG_MAX_K 65536   // centre indices are uint16 (0 .. 65535)
// Widest rows the screen serves: 96 K-steps of 16 dims, the wave's 32 rows held as MFMA operands in registers
#define KM_BIG_MAX_DIMS 1536
km_big_plan km_plan_big(int64_t n, int d, int k);
size_t km_big_x16_elems(const km_big_plan &pl);   // uint16 elements of the bf16 row operands
// candidate slots per half-row of the wide-row lists at d dims (16, 32 above 768 dims): cand holds 2 x this per row
int km_big_list_slot(int d);
size_t km_big_cop_elems(const km_big_plan &pl);   // uint16 elements of the bf16 centre operands
hipError_t km_launch_big_rows(const km_big_plan &pl, const float *X, int64_t n, int d, uint16_t *X16T, float *xsq,
                              hipStream_t s);
hipError_t km_launch_big_centres(const km_big_plan &pl, const float *C, int k, int d, float *csq, float *cn,
                                 uint16_t *Cop, float *maxes, km_control *ctl, const int32_t *stop, hipStream_t s);
// xmax: the largest |x|^2 over every slice (float bits), for the approximate mode's half-precision guard
hipError_t km_launch_big_xmax(const float *xsq, int64_t n, uint32_t *xmax, hipStream_t s);

// ---- empty-cluster relocation on the device (km_reloc.hip)
// Words of the selection state; blocks of the tie count (its size).
size_t km_reloc_state_words();
int64_t km_reloc_blocks(int64_t n, int cus);
// From the pass's totals tot (k, d + 2) and every row's label and best: the empty clusters (empties, k), the rows
// they take (sel, ord: k each), the patched float64 totals (ws, k (d + 2)) and the next centres Cn (k, d).
// part_X / part_rows: the slices in row order (copied into parts_dev, 16 bytes each). State word 5 holds the
// number of empty clusters afterwards.
hipError_t km_launch_relocate(const double *tot, int k, int d, int64_t n, const float *best, const uint32_t *labels,
                              const float *const *part_X, const int64_t *part_rows, int nparts, void *parts_dev,
                              uint32_t *st, int32_t *empties, int64_t *sel, int64_t *ord, uint32_t *tiecnt,
                              double *ws, float *Cn, int cus, hipStream_t s);
#define KM_RELOC_NEMPTY_WORD 5
// KM_APPROX approximates from KM_APPROX_MIN_DIMS dims while sqrt(max |x|^2 max |c|^2) < 65504 / 4; exact otherwise
#define KM_APPROX_MIN_DIMS 64
// sraw (may be null): the raw screen values a' of the tiles t with t % sstride == 0 (packed keys only),
// sraw[((t / sstride) nchunks + ch) 64 + lane][16], for the per-centre bounds' sample
hipError_t km_launch_big_screen(const km_big_plan &pl, int mode, const uint16_t *X16T, const float *xsq,
                                const uint32_t *xmax, int64_t n, int d, const uint16_t *Cop, const float *maxes, int k,
                                uint16_t *ncand, uint16_t *cand, uint32_t *over, uint32_t *multi, km_control *ctl,
                                const int32_t *stop, hipStream_t s, float *sraw = nullptr, int64_t sstride = 1);
// lite: the pass returns no per-row distances; single-candidate rows take their label without one. okeys: n words
// for the full scan of the overflow rows split over centre ranges (above 256 centres; null: one range)
// The rows loop for all n rows of a part, tiled (64 rows x 64 centres per block step, 32 dims at a time through
// LDS): the same labels and best, bit for bit, for rows too wide for one thread's registers (n < 2^32 - 64).
hipError_t km_launch_rows_tiled(const float *X, int64_t n, int d, const float *C, int k, uint32_t *labels, float *best,
                                const int32_t *stop, hipStream_t s);
hipError_t km_launch_big_rescore(const float *X, int64_t n, int d, const float *C, int k, const uint16_t *ncand,
                                 const uint16_t *cand, const uint32_t *over, const uint32_t *multi, km_control *ctl,
                                 uint32_t *labels, float *best, int lite, uint64_t *okeys, const int32_t *stop,
                                 hipStream_t s, const struct km_bnd_refresh *bref = nullptr);
// C_lite non-null: the best column is the rows' FMA-form distances to C, not best[] (pair with a lite rescore)
hipError_t km_launch_big_accum(const km_big_plan &pl, const float *X, int64_t n, int d, const uint32_t *labels,
                               const float *best, const float *C_lite, int k, uint32_t *H, uint32_t *counts,
                               uint32_t *base, uint32_t *perm, double *pieces, double *tmp, const int32_t *stop,
                               hipStream_t s);
// ---- per-centre lower bounds between passes (km_bounds.hip; the reference's Elkan bounds, core.py:1690-2015)
//
// For exact wide-row passes from KM_BND_MIN_DIMS dims: one float16 lower bound per (row, centre) on the distance
// |x - c| (not squared), kept between passes in a frame: the stored value less S_c, the centre's summed drift since
// the frame began, bounds sqrt(D_c) (1 - g) from below (g: the direct form's relative error). Per row an upper
// bound ub >= sqrt(D_l) (1 + g) on the distance to one centre l (ubl), raised by l's drift each pass. A pass on
// the bounds scores exactly only the centres whose bound is not above ub (the rows loop's label is always one of
// them), through the same candidate lists the screen fills.
// Layout of the bounds, tile-major like the screen's registers: km_bnd_index(row, c, nchunks).
#define KM_BND_MIN_DIMS 256          // the reference's BOUNDS_MIN_DIMS (core.py:513)
#define KM_BND_MIN_K 64              // the reference's TILES_MIN_K, which _bounds_ok requires (core.py:1722-1724)
#define KM_BND_MAX_BYTES ((size_t)16 << 30)   // the reference's BOUNDS_MAX_BYTES (core.py:515)
#define KM_BND_SAMPLE_TILES 64       // 32-row tiles the gate samples (2048 rows; the reference's BOUNDS_SAMPLE_ROWS is
                                     // 8192): each sampled tile re-reads every centre operand, so the sample's cost is
                                     // in proportion to its tiles, and 2048 rows x k centres estimate a fraction near
                                     // 5 % to well under a percent
__host__ __device__ inline int64_t km_bnd_index(int64_t row, int c, int nchunks) {
    const int ch = c >> 5, cc = c & 31;
    const int h = (cc >> 2) & 1, v = ((cc >> 3) << 2) | (cc & 3);
    return (((row >> 5) * nchunks + ch) * 64 + (row & 31) + 32 * h) * 16 + v;
}
// centre held at value v of half h of chunk ch (the screen's accumulator order)
__host__ __device__ inline int km_bnd_centre(int ch, int h, int v) { return 32 * ch + 8 * (v >> 2) + 4 * h + (v & 3); }

// The wide-row screen's error bound (km_big.hip explains it): |a'_c - A_c| <= E for every centre, from the row's |x|^2
// (rounded up) and |bf16(x) - x|, the centres' max |c|, max |c|^2 and max |bf16(-2c) + 2c|, and the constants of
// nacc = 16 DS + 2 accumulated terms (km_screen_consts); nx gets |x| rounded up.
__host__ __device__ constexpr double km_screen_gamma(int m) {
    return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08);
}
struct km_screen_k {
    float gacc, gam2, tiny;
};
__host__ __device__ constexpr km_screen_k km_screen_consts(int nacc) {
    return km_screen_k{(float)(2.04 * km_screen_gamma(nacc) * (1.0 + 0x1p-20)),
                       (float)((1.01 * km_screen_gamma(nacc) + 0x1p-16 + 0x1p-23) * (1.0 + 0x1p-20)),
                       (float)(nacc * 0x1p-118)};
}
__host__ __device__ inline float km_screen_E(float xsq_up, float exn, float cnmax, float csqmax, float fmax,
                                             km_screen_k q, float &nx) {
    nx = __builtin_sqrtf(xsq_up) * (1.0f + 0x1p-22f);
    return (2.0f * exn * cnmax + nx * fmax + exn * fmax) * (1.0f + 0x1p-20f) + q.gacc * nx * cnmax + q.gam2 * csqmax +
           (float)0x1p-119 * (nx + cnmax) + q.tiny;
}

struct km_bnd {
    int32_t skip_plain;    // nonzero: the plain screen stands down (bounds, a build, or the loop stopped)
    int32_t skip_bscreen;  // nonzero: the bound-writing screen stands down (bounds, or the loop stopped)
    int32_t skip_list;     // nonzero: the bounds list stands down (a screened pass, or the loop stopped)
    int32_t build;         // this pass writes every tile's bounds (else the sample tiles' only)
    int32_t sample_ok;     // the sample tiles have bounds from an earlier tracked pass
    int32_t built;         // every tile's bounds do (refreshes are worth writing)
    unsigned long long visits;     // sampled (row, centre) pairs this pass would visit, the ub centre excluded
    unsigned long long pairs;      // sampled (row, centre) pairs
    unsigned long long n_bounds;   // passes run on the bounds
    unsigned long long n_builds;   // passes that wrote every tile's bounds
    unsigned long long n_tracked;  // tracked passes
    double last_frac;              // the sampled fraction at the last tracked pass
};
// The bounds' slack factors for rows of d dims: lo <= 1 - g, hi >= 1 + g beyond float32 rounding
float km_bnd_lo(int d);
float km_bnd_hi(int d);
// Per pass, before the screen: each centre's drift |C - Clast| (rounded up) into delta and S (valid = 0 starts a
// new state: S = 0, nothing sampled, nothing built); Clast = C.
hipError_t km_launch_bnd_drift(const float *C, float *Clast, int k, int d, int valid, float *S, float *delta,
                               km_bnd *bs, const int32_t *stop, hipStream_t s);
// Per slice, the sample tiles (t % tstride == 0): the count of the pairs the stored bounds would visit now; then
// (once) the decision and the gates.
hipError_t km_launch_bnd_count(const uint16_t *lb, const float *ub, const uint32_t *ubl, int64_t n, int k,
                               int nchunks, int64_t tstride, const float *S, const float *delta, float hi,
                               km_bnd *bs, const int32_t *stop, hipStream_t s);
hipError_t km_launch_bnd_decide(km_bnd *bs, double max_visited, float *S, int k, const int32_t *stop, hipStream_t s);
// After a plain screen that wrote the sample tiles' raw screen values sraw (km_launch_big_screen with sraw): their
// bounds in the current frame and their rows' ub / ubl; gated on bs->skip_plain. ds: the screen's K-steps.
hipError_t km_launch_bnd_resample(const float *sraw, const float *xsq, int64_t n, int d, int ds, const float *maxes,
                                  int k, int nchunks, int64_t tstride, uint16_t *lb, float *ub, uint32_t *ubl,
                                  const float *S, km_bnd *bs, hipStream_t s);
// A pass on the bounds, one slice: candidate lists (ncand/cand/over/multi as the screen writes them) and every
// row's raised ub; gated on bs->skip_list.
hipError_t km_launch_bnd_list(const uint16_t *lb, float *ub, const uint32_t *ubl, int64_t n, int k, int nchunks,
                              const float *S, const float *delta, float hi, uint16_t *ncand, uint16_t *cand, int slot,
                              uint32_t *over, uint32_t *multi, km_control *ctl, km_bnd *bs, int cus, hipStream_t s);
// After the full scan of a slice's overflow rows: their ub from the exact best (when bs->built).
hipError_t km_launch_bnd_overfix(const uint32_t *over, const km_control *ctl, const uint32_t *labels,
                                 const float *best, float *ub, uint32_t *ubl, float hi, const km_bnd *bs,
                                 const int32_t *stop, hipStream_t s);
// Bound-writing screen (one slice) of a build: the screen's lists plus every row's ub / ubl and every tile's float16
// bounds; gated on bs->skip_bscreen.
hipError_t km_launch_big_screen_bnd(const km_big_plan &pl, const uint16_t *X16T, const float *xsq, int64_t n, int d,
                                    const uint16_t *Cop, const float *maxes, int k, uint16_t *ncand, uint16_t *cand,
                                    uint32_t *over, uint32_t *multi, km_control *ctl, uint16_t *lb, float *ub,
                                    uint32_t *ubl, km_bnd *bs, int cus, hipStream_t s);
// Refreshes the rescoring and the overflow fix write (null: none): the bounds of a slice, S, lo/hi
struct km_bnd_refresh {
    uint16_t *lb;        // the slice's bounds
    float *ub;           // the slice's upper bounds
    uint32_t *ubl;
    const float *S;
    int nchunks;
    float lo, hi;
    const km_bnd *bs;    // refreshes only when bs->built
};
// ---- per-cluster sums over rows listed in cluster order, in fixed chunks (km_chunks.hip)
#define KM_CHUNK_MAX_DIMS 1536
// pieces for npos listed positions: mode 0 (rows, best[] column) and 1 (rows, distances to C), mode 2 (change
// entries)
int64_t km_chunk_piece_doubles(int64_t npos, int d, int mode);
// The k (d + 2) sums into tmp: [count, best column, x] per cluster, from the positions perm lists in label order
// (counts / base per label). Modes 0 / 1: rows of X (perm holds row indices; lab, best per row; npos rows).
// Mode 2: change entries (perm holds entry indices; lab, erow per entry, rows found in the device slice table;
// 2 *npos_dev positions). gate (may be null): nonzero skips the work.
hipError_t km_launch_chunk_sums(int mode, const float *X, const km_slice *slices, int nslices, int d,
                                const uint32_t *lab, const uint32_t *erow, const float *best, const float *C,
                                const uint32_t *perm, const uint32_t *counts, const uint32_t *base, int k,
                                const uint32_t *npos_dev, int64_t npos, double *pieces, double *tmp,
                                const int32_t *gate, hipStream_t s);
// The counting sort by label and per-cluster float64 sums in row order for any rows path (d <= 1536): rows whose
// labels and best are known. H holds km_sorted_blocks(n) x k counters; tmp receives the k (d + 2) range sums.
int64_t km_sorted_blocks(int64_t n);
// The stable counting sort by label alone: perm lists 0 .. n-1 grouped by label (ascending), ascending within a
// label; counts / base the k group sizes and starts. H holds km_sorted_blocks(n) x k counters. half (device, may
// be null): sort only the first 2 *half labels.
hipError_t km_launch_label_sort(const uint32_t *labels, int64_t n, int k, uint32_t *H, uint32_t *counts,
                                uint32_t *base, uint32_t *perm, const int32_t *stop, hipStream_t s,
                                const uint32_t *half = nullptr);
hipError_t km_launch_sorted_accum(const float *X, int64_t n, int d, const uint32_t *labels, const float *best, int k,
                                  uint32_t *H, uint32_t *counts, uint32_t *base, uint32_t *perm, double *pieces,
                                  double *tmp, const int32_t *stop, hipStream_t s);
// Centres above which the rows path accumulates through the counting sort (the generic accumulation re-reads the
// rows once per block of clusters)
#define KM_SORTED_MIN_K 4096
