/*
 * kmeans_hip.h - C ABI of libkmeans_hip.so, the MI355X (gfx950) engine for the exact Lloyd pass.
 *
 * Plain pointers and sizes only. Every entry point returns KM_OK (0) or a negative code; the message for the
 * last failure on a context is km_last_error(ctx). Each context owns one HIP stream (default priority), its
 * device copies of the data and its workspaces; calls on one context must not overlap (one context per host
 * thread). Citations name the reference (kakollu/mlx-kmeans) interface each entry point replaces.
 *
 * Data layout: rows are float32, row-major (rows, dims), C-contiguous - the reference's layout
 * (mlx_kmeans/estimator.py:120). Centres are float32 (k, dims). Totals are float64 (k, dims + 2) in the
 * reference's column order [count, sum of best distance, sum of x_0 .. x_{dims-1}] (core.py:1629-1636).
 *
 * Exactness contract (mode KM_EXACT): every label is the centre with the smallest float32 distance
 * s = sum_j (x_j - c_j)^2, accumulated for j ascending with the product and the add rounded separately,
 * lowest index on an exact tie (the rows loop, core.py:263-274); best is that s. Whatever kernel path runs,
 * the labels and best values are these, bit for bit. Mode KM_APPROX (exact=False, estimator.py:18-30): on the
 * wide-row path (16 < dims <= 1536, k <= 4096, k * dims >= 1024) the label is the bf16 screen's minimiser, taken on
 * trust, and best is the exact distance above to that label; every other path is exact in either mode.
 */
#ifndef KMEANS_HIP_H
#define KMEANS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct km_ctx km_ctx;

/* return codes */
#define KM_OK 0
#define KM_EINVAL (-1)      /* bad argument: the message carries the reference's wording where one exists */
#define KM_EDEVICE (-2)     /* a HIP call or a kernel launch failed */
#define KM_ENOMEM (-3)      /* device allocation failed */
#define KM_ENODATA (-4)     /* no data set on the context */

/* where a pointer argument lives */
#define KM_HOST 0
#define KM_DEVICE 1

/* assignment mode: exact=True / exact=False of the reference's KMeans (estimator.py:67-69) */
#define KM_EXACT 0
#define KM_APPROX 1

/* kernel path, the reference's `method` argument (core.py:2018): AUTO picks by shape */
#define KM_PATH_AUTO 0
#define KM_PATH_ROWS 1      /* direct-form scan of every centre on the vector ALUs (the reference's "rows") */
#define KM_PATH_MFMA 2      /* bf16 matrix-core screen + exact rescoring of the candidates (the reference's "tiles") */
#define KM_PATH_FUSED 3     /* dims <= 16: the rows loop fused with the accumulation, one read of the rows (the
                             * reference's single-read "fused" / "onehot" kernels, core.py:1478-1534, 1562-1675) */

/* Create a context on HIP device `device` (ordinal). NULL on failure (no context to carry a message).
 * Replaces the reference's module-global per-dataset caches (core.py:548-578): all state lives here. */
km_ctx *km_create(int32_t device);

/* Free every device buffer and the stream. NULL is accepted. */
void km_destroy(km_ctx *ctx);

/* Message for the last failure on ctx ("" if none). Valid until the next call on ctx. */
const char *km_last_error(const km_ctx *ctx);

/* Set the data to one slice of `rows` x `dims` float32. where = KM_HOST copies it to the device (the
 * context owns the copy); where = KM_DEVICE borrows a device pointer, which must stay valid and unchanged
 * until the data is replaced or the context destroyed. Replaces KMeans._parts (estimator.py:108-125). */
int32_t km_set_data(km_ctx *ctx, const float *X, int64_t rows, int32_t dims, int32_t where);

/* Append one more slice with the same dims (the reference's list-of-slices input, estimator.py:110-111).
 * Totals are summed over slices; labels come back concatenated in slice order. */
int32_t km_append_data(km_ctx *ctx, const float *X, int64_t rows, int32_t where);

/* Total rows over all slices, and dims (0 if no data). */
int64_t km_rows(const km_ctx *ctx);
int32_t km_dims(const km_ctx *ctx);

/* One assignment pass with centres C (host, k x dims) and no update.
 *   totals: host (k, dims+2) float64, required.
 *   labels: host uint32 per row, or NULL.   best: host float32 per row, or NULL.
 * Replaces _gpu_pass (core.py:2018-2197), which assign_mlx (core.py:2200-2206) wraps. */
int32_t km_pass(km_ctx *ctx, const float *C, int32_t k, int32_t mode, int32_t path, double *totals,
                uint32_t *labels, float *best);

/* One Lloyd iteration from centres C (host, k x dims): C_out (host, k x dims) gets the new centres,
 * *inertia the inertia of C (before the update), *n_empty the number of clusters that came up empty and
 * were relocated as scikit-learn does. Replaces lloyd_step (core.py:2209-2242). */
int32_t km_lloyd_step(km_ctx *ctx, const float *C, int32_t k, int32_t mode, int32_t path, float *C_out,
                      double *inertia, int32_t *n_empty);

/* Up to max_iter Lloyd iterations from C0 (host, k x dims) with the reference's stopping rule
 * |prev - inertia| <= tol * prev (estimator.py:147-149; a negative tol never stops a loop with inertia > 0),
 * spherical renormalisation when spherical != 0 (estimator.py:127-130, 141-142). Iterations run back to back on the device; the host looks at the
 * device-side state only every few iterations and when a cluster empties. Outputs (host): C_out the final
 * centres, *last_inertia the inertia reported by the last iteration, *n_iter the iterations run,
 * *n_relocated the total empty clusters relocated. Replaces KMeans._one_run's loop (estimator.py:132-150). */
int32_t km_fit(km_ctx *ctx, const float *C0, int32_t k, int32_t max_iter, double tol, int32_t mode,
               int32_t spherical, float *C_out, double *last_inertia, int32_t *n_iter, int32_t *n_relocated);

/* Greedy k-means++ seeding on a sample of the rows, every round on the device (replaces kmeans_pp_init,
 * core.py:153-192, and its kernels core.py:70-106). sample: m ascending global row indices (host; the reference
 * draws them with rng.choice(rows, m, replace=False), sorted); first: the first pick, an index into the sample;
 * seeds: k - 1 per-round seeds (host; the reference's rng.integers(2**63 - 1, size=k - 1)). Round r keeps, of
 * 2 + floor(ln k) candidates drawn with probability proportional to the squared distance to the nearest pick so
 * far (candidate t: the row with the largest d2 / (-ln u), u from splitmix64(seed_r ^ splitmix64(i * trials + t))),
 * the one that lowers the summed squared distance the most (first on a tie). C_out (host, k x dims): the picked
 * rows in pick order. Requires m >= k and 2 + floor(ln k) <= 16. The context keeps two device copies of the
 * sample (dims x m and m x dims float32) and the rounds' minima (two trials x m float32 arrays). */
int32_t km_seed_pp(km_ctx *ctx, int32_t k, const int64_t *sample, int64_t m, int64_t first, const uint64_t *seeds,
                   float *C_out);

/* No counterpart in the reference: an allocation-free km_pass for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). One exact assignment pass over
 * device rows X (rows x dims float32, row-major) with device centres C (k x dims): totals (device, k x (dims + 2)
 * float64, the km_pass layout), labels (device uint32 per row) and best (device float32 per row) - all required -
 * get km_pass's results (labels and best the same bits; totals from the same kernel family, summed over a
 * number of row blocks that fits the scratch). Launches on `stream` (a hipStream_t; NULL is the null stream) and
 * returns without waiting. It allocates nothing: its workspaces are the library's static device scratch array,
 * 32 MiB per device, which every call on that device shares and which keeps the last call's contents - calls that
 * overlap on one device race. Shapes whose partials would not fit it even as a single block (16 bytes per entry:
 * k * (dims + 2) above about 2.09 million) are refused with KM_EINVAL before anything is launched. The wide-row path (16 < dims <= 1536
 * in km_pass) needs a bf16 copy of the rows and is not used: those shapes run the rows path. ctx supplies the
 * device, the scratch address and the error message; its own data and buffers are not touched. */
int32_t km_pass_noalloc(km_ctx *ctx, const float *X, int64_t rows, int32_t dims, const float *C, int32_t k,
                        double *totals, uint32_t *labels, float *best, void *stream);

/* Per-centre lower bounds between Lloyd passes (the reference's Elkan bounds, core.py:1690-2015). Exact passes on the
 * wide-row path from 256 dims and 64 centres keep, per (row, centre), a float16 lower bound on the distance and per
 * row an upper bound, and run a pass on them (exact scoring of only the centres a bound cannot rule out; the same
 * labels and best, bit for bit) when a strided sample of 2048 rows says at most max_visited of the (row, centre)
 * pairs need scoring - the reference's gate BOUNDS_MAX_VISITED (core.py:516, 2063-2106). km_bounds sets that
 * fraction for ctx (default 0.05; 0 turns the bounds off and frees nothing until the data changes).
 * km_bounds_info reports, since the data was set: passes tracked, passes run on the bounds, passes that wrote
 * every row's bounds (the reference's build, core.py:2091-2096), and the sampled fraction of the last tracked pass
 * (the reference's "visited", core.py:2010). Any pointer may be NULL. */
int32_t km_bounds(km_ctx *ctx, double max_visited);
int32_t km_bounds_info(km_ctx *ctx, int64_t *passes_tracked, int64_t *passes_on_bounds, int64_t *builds,
                       double *last_fraction);

/* Kernel timing with HIP events on the context's stream. km_profile(ctx, 1) clears and starts recording;
 * km_profile_read gives, for kernel id `kernel`, the summed milliseconds and launch count so far.
 * km_kernel_name(id) names an id ("" past the last); ids are stable within one build. */
int32_t km_profile(km_ctx *ctx, int32_t enable);
int32_t km_profile_read(km_ctx *ctx, int32_t kernel, double *ms_total, int64_t *launches);
const char *km_kernel_name(int32_t kernel);

/* Per-pass times, in milliseconds, of the km_fit loops run since km_profile(ctx, 1): one HIP event at every pass
 * boundary on the context's stream. Copies up to cap of them into ms (may be null) and returns how many there
 * are. The reference times whole fits from the host (bench.py); this reads each pass of one. */
int64_t km_profile_passes(km_ctx *ctx, double *ms, int64_t cap);

/* Streaming-read probe: the device's HBM read rate for a plain kernel over a fresh `bytes`-byte array (a
 * multiple of 16, at least 16 MiB), the median of `reps` launches for each of a few grid sizes, the best of
 * them in GB/s. Replaces quick_bench.py:48-63 (stream_rate), the floor the reference's pass times are read
 * against. Allocates and frees the array. */
int32_t km_stream_probe(km_ctx *ctx, int64_t bytes, int32_t reps, double *gbps);

/* Which path the last pass on ctx ran for its assignment (KM_PATH_ROWS, _MFMA or _FUSED), and the number of
 * rows in that pass the matrix-core screen could not settle alone: on the fused path (16 to 64 dims) rows with
 * more than one centre inside the error window (or non-finite rows), scored against every centre; on the
 * wide-row path rows that took the full scan of every centre (more than 16 centres in a half-row's window,
 * 32 above 768 dims, or non-finite data). 0 on the other paths. */
int32_t km_last_path(const km_ctx *ctx);
int64_t km_last_fallback_rows(km_ctx *ctx);

/* ABI version of this header. */
int32_t km_version(void);

#ifdef __cplusplus
}
#endif

#endif
