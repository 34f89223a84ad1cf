// libkmeans_hip.so: the C ABI (include/kmeans_hip.h) and the host runtime around the kernels.
//
// A context owns one HIP stream, the device copies (or borrowed pointers) of the data slices, two centre buffers,
// and every workspace of a pass. A Lloyd iteration is three kernels on that stream:
//   assignment + accumulation into per-block partials (fused MFMA, fused rows, or the generic pair)
//   ->  k_reduce_split (float64 sums of fixed ranges of partials)
//   ->  k_finish (totals; new centres into the other buffer; in its last block the statistics and stopping rule)
// Pass p reads centre buffer p % 2 and writes buffer (p + 1) % 2. The loop state lives in a device-side
// km_control block and every kernel of a pass is gated on it, so km_fit queues iterations back to back and looks
// at the state only every KM_FIT_BATCH iterations. A pass that leaves clusters empty stops the queue; the device
// then relocates them the way the reference's lloyd_step does (core.py:2222-2242), from that pass's input
// centres and totals, and the loop resumes.
#include "kmeans_hip.h"
#include "km_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <vector>

#define KM_ABI_VERSION 1
static const int KM_FIT_BATCH = 8;
// In the fit loop a pass that accumulates only changed rows adds its (float32 fused, float64 wide-row) change sums
// to the previous totals; every KM_REANCHOR_PASSES passes after a recording pass, one pass records every row again,
// so the totals never carry more than that many passes of change rounding.
static const int KM_REANCHOR_PASSES = 32;
// The fused path's change-only passes use the kernel without candidate lists (open rows scanned by the whole
// wave) while the context's last fit left at most this fraction of rows open: then about 0.1 % of 64-row blocks
// hold more than four open rows (where the lists start to pay).
static const double KM_SCAN_ONLY_FRAC = 0.01;

template <class T>
struct DBuf {
    T *p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t n) {
        if (n <= cap && p) return hipSuccess;
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
        if (n == 0) n = 1;
        hipError_t e = hipMalloc((void **)&p, n * sizeof(T));
        if (e == hipSuccess) cap = n;
        else p = nullptr;
        return e;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

struct Part {
    const float *X;   // device pointer used by kernels
    float *owned;     // non-null when the context allocated X
    int64_t rows;
    bool aligned;     // 16-byte aligned: whole-float4 row loads are allowed
    uint16_t *x16 = nullptr;   // the wide-row path's bf16 row operands (built on first use)
    float *xsq = nullptr;      // |x|^2 rounded up per row (built with x16)
    int x16_ds = 0;            // K-steps x16 was built for
};

// Which kernel family ran a pass (the public path code is coarser: both MFMA families report KM_PATH_MFMA).
enum km_family { FAM_NONE = 0, FAM_ROWS, FAM_MFMA_FUSED, FAM_LOWD, FAM_BIG };

struct ProfRec {
    int kernel;
    hipEvent_t a, b;
};

struct km_ctx {
    int device = 0;
    km_device_info dev{256, 65536};
    hipStream_t stream = nullptr;
    std::vector<Part> parts;
    int32_t d = 0;
    int64_t n = 0;
    char err[1024] = {0};   // message of the last failure (a fixed buffer: reporting allocates nothing)
    int32_t last_path = 0;
    int last_family = FAM_NONE;
    DBuf<uint16_t> cop;     // wide-row path: bf16 centre operands
    DBuf<float> bcsq, bcn, bmax;
    DBuf<uint16_t> ncand;
    DBuf<uint16_t> cand;
    DBuf<uint32_t> hist, counts, base, perm, over, multi;
    DBuf<uint64_t> okeys;   // wide-row path: the overflow rows' (best, label) keys of the split full scan
    DBuf<uint32_t> xmax;    // wide-row path: the largest |x|^2 over every slice (float bits)
    DBuf<uint8_t> lstate;   // the fit loop's label of every row (one byte; each slice at lstate_off[i])
    std::vector<int64_t> lstate_off;
    DBuf<float> Cb[2];      // centre buffers (k, d): pass p reads Cb[p & 1], writes Cb[(p + 1) & 1]
    DBuf<float> psum, pcomp;
    DBuf<uint32_t> pmask;   // change-only fused passes: per row-block, the clusters whose partials it wrote
    DBuf<double> tot;
    DBuf<double> tot2;      // (k, 2) [count, best] totals recomputed for km_pass on the fused path
    DBuf<double> red;       // range sums of the reduce (S, k * (d + 2))
    DBuf<uint32_t> labels;
    DBuf<float> best;
    DBuf<float> pp_S, pp_R, pp_C;   // k-means++: the row sample (transposed, dims x m; and rows, m x dims) and
                                    // the picked rows
    DBuf<int64_t> pp_idx;       // k-means++: the sample's row indices, local to their slice
    DBuf<uint32_t> rl_st, rl_tie;   // relocation: selection state and per-block tie counts
    DBuf<int32_t> rl_empty;         // relocation: the empty clusters, ascending
    DBuf<int64_t> rl_sel;           // relocation: the taken rows, then in order
    DBuf<double> rl_ws;             // relocation: the patched totals
    DBuf<char> rl_parts;            // relocation: the slice table
    DBuf<char> pp_ws;           // k-means++: the rounds' workspace
    // change-only accumulation of the wide-row fit loop: labels alternate between `labels` (even passes) and
    // wlab (odd passes), each pass compared with the other
    DBuf<uint32_t> wlab;
    DBuf<uint32_t> wd_bcnt, wd_e;   // per-block change counts + m; the entry arrays (elab, erow: wd_limit each x2)
    DBuf<uint32_t> wd_H, wd_cnt, wd_base, wd_perm;   // the entries' counting sort by label
    DBuf<int32_t> wd_gate;          // [0] nonzero: no change-only sums this pass; [1] nonzero: no full accumulation
    DBuf<double> wd_part, wd_mu;    // mean / scatter partials; [mu (d), T] of the data set
    DBuf<double> pieces;            // the sums of clusters whose sorted rows span several chunks, per chunk
    DBuf<km_slice> wd_slices;       // the slice table on the device
    // per-centre bounds between exact wide-row passes (km_bounds.hip): the float16 lower bounds (each slice's
    // from bnd_off[i]), every row's upper bound and its centre, each centre's summed drift S, this pass's drift,
    // the previous tracked pass's centres, and the device-side state (gates, sample count, counters)
    DBuf<uint16_t> bnd_lb;
    DBuf<float> bnd_ub, bnd_S, bnd_delta, bnd_Clast;
    DBuf<uint32_t> bnd_ubl;
    DBuf<km_bnd> bnd_st;
    DBuf<float> bnd_raw;            // the sample tiles' raw screen values (a screened pass's resample reads them)
    std::vector<int64_t> bnd_off, bnd_soff;   // per slice: its first bound, its first sample tile
    bool bnd_valid = false;         // the device state describes this data and bnd_k
    int bnd_k = 0;
    double bnd_max_visited = 0.05;  // the reference's BOUNDS_MAX_VISITED (core.py:516); 0 turns the bounds off
    double open_frac = -1.0;        // rows the fused screen left open, per row and pass, in this context's last fit
                                    // on that path (< 0: none yet)
    std::vector<km_slice> wd_slices_h;
    bool wd_ready = false;          // wd_mu and wd_slices describe the current data
    int64_t wd_limit = 0;           // the most changed rows a change-only pass takes
    km_control *ctl = nullptr;    // device
    km_control *ctl_h = nullptr;  // pinned host mirror
    unsigned char *scratch = nullptr;   // device address of this device's copy of `scratch` (km_pass_noalloc)
    bool prof = false;
    std::vector<ProfRec> recs;
    std::vector<hipEvent_t> pool;
    double prof_ms[KK_COUNT] = {};
    int64_t prof_n[KK_COUNT] = {};
    std::vector<double> pass_ms;   // per-pass times of the fit loops run while timing is on
};

static int fail(km_ctx *c, int code, const char *fmt, ...) {
    if (!c) return code;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->err, sizeof c->err, fmt, ap);
    va_end(ap);
    return code;
}

#define HIPCHK(ctx, expr)                                                                                 \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess)                                                                             \
            return fail((ctx), e_ == hipErrorOutOfMemory ? KM_ENOMEM : KM_EDEVICE, "%s failed: %s (%s:%d)", \
                        #expr, hipGetErrorString(e_), __FILE__, __LINE__);                                \
    } while (0)

static hipEvent_t get_event(km_ctx *c) {
    if (!c->pool.empty()) {
        hipEvent_t e = c->pool.back();
        c->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Launch through f, bracketed by events on the context's stream when timing is on.
template <class F>
static hipError_t launch(km_ctx *c, int kid, F &&f) {
    if (!c->prof) return f();
    hipEvent_t a = get_event(c), b = get_event(c);
    if (!a || !b) return f();
    (void)hipEventRecord(a, c->stream);
    hipError_t e = f();
    (void)hipEventRecord(b, c->stream);
    c->recs.push_back({kid, a, b});
    return e;
}

static void harvest(km_ctx *c) {
    if (c->recs.empty()) return;
    (void)hipStreamSynchronize(c->stream);
    for (auto &r : c->recs) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            c->prof_ms[r.kernel] += ms;
            c->prof_n[r.kernel] += 1;
        }
        c->pool.push_back(r.a);
        c->pool.push_back(r.b);
    }
    c->recs.clear();
}

// ------------------------------------------------------------------ the allocation-free pass's scratch
//
// km_pass_noalloc works in this array only: its control block, per-block partials and range sums. Every device
// the library runs on holds its own copy until the process ends; km_create looks up the copy's device address
// with that device current and keeps it in the context (the array's name in host code is a host-side stand-in,
// not a device address). Calls that overlap on one device share the array and race.
#define KM_SCRATCH_BYTES ((size_t)32 << 20)
static __device__ __align__(256) unsigned char scratch[KM_SCRATCH_BYTES];

// ------------------------------------------------------------------ context and data

extern "C" km_ctx *km_create(int32_t device) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return nullptr;
    if (hipSetDevice(device) != hipSuccess) return nullptr;
    km_ctx *c = new km_ctx();
    c->device = device;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
        if (prop.multiProcessorCount > 0) c->dev.cus = prop.multiProcessorCount;
        if (prop.sharedMemPerBlock > 0) c->dev.lds_max = (size_t)prop.sharedMemPerBlock;
    }
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return nullptr;
    }
    if (hipMalloc((void **)&c->ctl, sizeof(km_control)) != hipSuccess ||
        hipHostMalloc((void **)&c->ctl_h, sizeof(km_control), hipHostMallocDefault) != hipSuccess) {
        if (c->ctl) (void)hipFree(c->ctl);
        (void)hipStreamDestroy(c->stream);
        delete c;
        return nullptr;
    }
    memset(c->ctl_h, 0, sizeof(km_control));
    // this device's copy of the allocation-free pass's scratch (the device is current here)
    void *sp = nullptr;
    if (hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)) == hipSuccess) c->scratch = (unsigned char *)sp;
    return c;
}

static void drop_parts(km_ctx *c) {
    for (auto &p : c->parts) {
        if (p.owned) (void)hipFree(p.owned);
        if (p.x16) (void)hipFree(p.x16);
        if (p.xsq) (void)hipFree(p.xsq);
    }
    c->parts.clear();
    c->n = 0;
    c->d = 0;
    c->wd_ready = false;
    c->bnd_valid = false;
}

extern "C" void km_destroy(km_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    drop_parts(c);
    c->Cb[0].release();
    c->Cb[1].release();
    c->psum.release();
    c->pcomp.release();
    c->tot.release();
    c->tot2.release();
    c->cop.release();
    c->bcsq.release();
    c->bcn.release();
    c->bmax.release();
    c->ncand.release();
    c->cand.release();
    c->hist.release();
    c->counts.release();
    c->base.release();
    c->perm.release();
    c->over.release();
    c->multi.release();
    c->okeys.release();
    c->xmax.release();
    c->lstate.release();
    c->red.release();
    c->labels.release();
    c->best.release();
    c->pp_S.release();
    c->pp_R.release();
    c->pp_C.release();
    c->pp_idx.release();
    c->pp_ws.release();
    c->wlab.release();
    c->bnd_lb.release();
    c->bnd_ub.release();
    c->bnd_S.release();
    c->bnd_delta.release();
    c->bnd_Clast.release();
    c->bnd_ubl.release();
    c->bnd_st.release();
    c->bnd_raw.release();
    c->wd_bcnt.release();
    c->wd_e.release();
    c->wd_H.release();
    c->wd_cnt.release();
    c->wd_base.release();
    c->wd_perm.release();
    c->pieces.release();
    c->wd_gate.release();
    c->wd_part.release();
    c->wd_mu.release();
    c->wd_slices.release();
    c->rl_st.release();
    c->rl_tie.release();
    c->rl_empty.release();
    c->rl_sel.release();
    c->rl_ws.release();
    c->rl_parts.release();
    for (auto &r : c->recs) {
        (void)hipEventDestroy(r.a);
        (void)hipEventDestroy(r.b);
    }
    for (auto e : c->pool) (void)hipEventDestroy(e);
    if (c->ctl) (void)hipFree(c->ctl);
    if (c->ctl_h) (void)hipHostFree(c->ctl_h);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

extern "C" const char *km_last_error(const km_ctx *c) { return c ? c->err : "no context"; }

static int add_part(km_ctx *c, const float *X, int64_t rows, int32_t where) {
    if (!X) return fail(c, KM_EINVAL, "data pointer is null");
    if (rows < 1) return fail(c, KM_EINVAL, "expected a nonempty 2-D (rows, dims) array, got %lld rows", (long long)rows);
    Part p;
    p.X = nullptr;
    p.owned = nullptr;
    p.rows = rows;
    p.aligned = true;
    if (where == KM_DEVICE) {
        p.X = X;
        p.aligned = ((uintptr_t)X % 16) == 0;
    } else if (where == KM_HOST) {
        const size_t bytes = (size_t)rows * c->d * sizeof(float);
        HIPCHK(c, hipMalloc((void **)&p.owned, bytes));
        hipError_t e = hipMemcpyAsync(p.owned, X, bytes, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            (void)hipFree(p.owned);
            return fail(c, KM_EDEVICE, "copying the data to the device failed: %s", hipGetErrorString(e));
        }
        p.X = p.owned;
    } else {
        return fail(c, KM_EINVAL, "where must be KM_HOST or KM_DEVICE");
    }
    c->parts.push_back(p);
    c->n += rows;
    c->wd_ready = false;
    c->open_frac = -1.0;   // the open-row rate was the previous data's
    return KM_OK;
}

extern "C" int32_t km_set_data(km_ctx *c, const float *X, int64_t rows, int32_t dims, int32_t where) {
    if (!c) return KM_EINVAL;
    HIPCHK(c, hipSetDevice(c->device));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    drop_parts(c);
    if (dims < 1) return fail(c, KM_EINVAL, "expected a nonempty 2-D (rows, dims) array, got %d dims", dims);
    c->d = dims;
    int r = add_part(c, X, rows, where);
    if (r != KM_OK) c->d = 0;
    return r;
}

extern "C" int32_t km_append_data(km_ctx *c, const float *X, int64_t rows, int32_t where) {
    if (!c) return KM_EINVAL;
    if (c->parts.empty()) return fail(c, KM_ENODATA, "no data: call km_set_data first");
    HIPCHK(c, hipSetDevice(c->device));
    return add_part(c, X, rows, where);
}

extern "C" int64_t km_rows(const km_ctx *c) { return c ? c->n : 0; }
extern "C" int32_t km_dims(const km_ctx *c) { return c ? c->d : 0; }
extern "C" int32_t km_version(void) { return KM_ABI_VERSION; }
extern "C" int32_t km_last_path(const km_ctx *c) { return c ? c->last_path : 0; }

extern "C" int64_t km_last_fallback_rows(km_ctx *c) {
    if (!c) return -1;
    if (hipMemcpyAsync(c->ctl_h, c->ctl, sizeof(km_control), hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
        hipStreamSynchronize(c->stream) != hipSuccess)
        return -1;
    return (int64_t)c->ctl_h->fallback_rows;
}

// ------------------------------------------------------------------ one pass

static int check_centres(km_ctx *c, const float *C, int32_t k) {
    if (c->parts.empty()) return fail(c, KM_ENODATA, "no data: call km_set_data first");
    if (!C) return fail(c, KM_EINVAL, "centres pointer is null");
    if (k < 1) return fail(c, KM_EINVAL, "n_clusters must be a positive integer");
    return KM_OK;
}

// Decide the assignment path for this shape: the matrix-core screen once a row's distance work is large
// enough to hide its epilogue, the fused single-read scan for narrow rows, the generic two-kernel rows path
// otherwise. An explicit path that does not serve the shape is an error (-1).
static bool parts_aligned(const km_ctx *c) {
    for (auto &p : c->parts)
        if (!p.aligned) return false;
    return true;
}

static bool big_ok(const km_ctx *c, int k) {
    for (auto &p : c->parts)
        if (!km_plan_big(p.rows, c->d, k).ok) return false;
    return !c->parts.empty();
}

// Returns the kernel family for this pass (FAM_*), or -1 when an explicit path does not serve the shape.
static int choose_path(km_ctx *c, int k, int path, km_mfma_plan *mp) {
    const bool al = parts_aligned(c);
    *mp = km_plan_mfma(c->dev, c->n, c->d, k);
    if (!al) mp->ok = 0;
    const bool lowd_ok = km_plan_lowd(c->dev, c->n, c->d, k, al).ok != 0;
    const bool wide_ok = big_ok(c, k);
    if (path == KM_PATH_ROWS) return FAM_ROWS;
    if (path == KM_PATH_MFMA) return mp->ok ? FAM_MFMA_FUSED : wide_ok ? FAM_BIG : -1;
    if (path == KM_PATH_FUSED) return lowd_ok ? FAM_LOWD : -1;
    if (mp->ok && c->d >= 16 && (int64_t)k * c->d >= 192) return FAM_MFMA_FUSED;
    if (lowd_ok) return FAM_LOWD;
    if (wide_ok && (int64_t)k * c->d >= 1024) return FAM_BIG;
    return FAM_ROWS;
}

static int32_t family_path(int fam) {
    return fam == FAM_ROWS ? KM_PATH_ROWS : fam == FAM_LOWD ? KM_PATH_FUSED : KM_PATH_MFMA;
}

// Sizes the per-pass workspaces. Returns KM_OK or an error.
static int ensure_pass_buffers(km_ctx *c, int k, size_t total_rb, bool need_rows_scratch) {
    const int64_t kw = (int64_t)k * (c->d + 2);
    HIPCHK(c, c->psum.ensure(total_rb * (size_t)kw));
    HIPCHK(c, c->pcomp.ensure(total_rb * (size_t)kw));
    HIPCHK(c, c->tot.ensure((size_t)kw));
    HIPCHK(c, c->red.ensure((size_t)km_reduce_splits((int)total_rb, kw, c->dev.cus) * kw));
    if (need_rows_scratch) {
        HIPCHK(c, c->labels.ensure((size_t)c->n));
        HIPCHK(c, c->best.ensure((size_t)c->n));
    }
    return KM_OK;
}

// Partials -> totals in c->tot, and with KM_FIN_UPDATE the new centres into Cb[(pass + 1) & 1] and the pass
// statistics into the control block. presummed > 0: c->red already holds that many range sums.
static int finish_pass(km_ctx *c, int k, int rb, int pass, double tol, int flags, const int32_t *stop,
                       int presummed = 0, const int32_t *dsel = nullptr, const uint32_t *pmask = nullptr) {
    const int d = c->d;
    const int64_t kw = (int64_t)k * (d + 2);
    float *Cn = c->Cb[(pass + 1) & 1].p;
    if (!presummed) {
        const int S = km_reduce_splits(rb, kw, c->dev.cus);
        HIPCHK(c, launch(c, KK_REDUCE, [&] {
            return km_launch_reduce_finish(c->psum.p, c->pcomp.p, rb, kw, S, c->red.p, k, d, c->tot.p, Cn, c->ctl, pass,
                                           tol, flags, stop, c->stream, pmask);
        }));
        return KM_OK;
    }
    HIPCHK(c, launch(c, KK_FINISH, [&] {
        return km_launch_finish(c->red.p, presummed, k, d, c->tot.p, Cn, c->ctl, pass, tol, flags, stop, c->stream,
                                dsel ? c->Cb[pass & 1].p : nullptr, dsel ? c->wd_mu.p : nullptr, dsel);
    }));
    return KM_OK;
}

// Per-centre bounds for this wide-row pass: offered to exact passes from KM_BND_MIN_DIMS dims and KM_BND_MIN_K
// centres with packed keys, within KM_BND_MAX_BYTES of float16 bounds (the reference's _bounds_ok, core.py:1722-1724),
// unless turned off. Sizes the state (a new data set or k starts it again) and returns whether the pass is tracked,
// with the sample stride.
static int prepare_bounds(km_ctx *c, int k, int mode, const km_big_plan &bp0, bool *use, int64_t *tstride) {
    *use = false;
    if (c->bnd_max_visited <= 0.0 || mode != KM_EXACT || c->d < KM_BND_MIN_DIMS || k < KM_BND_MIN_K || bp0.ib <= 0)
        return KM_OK;
    int64_t tiles = 0, elems = 0;
    std::vector<int64_t> off;
    for (auto &p : c->parts) {
        const int64_t t = (p.rows + 31) / 32;
        off.push_back(elems);
        tiles += t;
        elems += t * bp0.nchunks * 1024;
    }
    if ((size_t)elems * sizeof(uint16_t) > KM_BND_MAX_BYTES) return KM_OK;
    if (c->bnd_k != k || off != c->bnd_off) c->bnd_valid = false;
    if (!c->bnd_valid) {
        HIPCHK(c, c->bnd_lb.ensure((size_t)elems));
        HIPCHK(c, c->bnd_ub.ensure((size_t)c->n));
        HIPCHK(c, c->bnd_ubl.ensure((size_t)c->n));
        HIPCHK(c, c->bnd_S.ensure((size_t)k));
        HIPCHK(c, c->bnd_delta.ensure((size_t)k));
        HIPCHK(c, c->bnd_Clast.ensure((size_t)k * c->d));
        HIPCHK(c, c->bnd_st.ensure(1));
        HIPCHK(c, hipMemsetAsync(c->bnd_st.p, 0, sizeof(km_bnd), c->stream));
        c->bnd_off = off;
        c->bnd_k = k;
    }
    *tstride = std::max<int64_t>(1, tiles / KM_BND_SAMPLE_TILES);
    c->bnd_soff.clear();
    int64_t stiles = 0;
    for (auto &p : c->parts) {
        c->bnd_soff.push_back(stiles);
        stiles += ((p.rows + 31) / 32 + *tstride - 1) / *tstride;
    }
    HIPCHK(c, c->bnd_raw.ensure((size_t)stiles * bp0.nchunks * 1024));
    *use = true;
    return KM_OK;
}

// A tracked pass: each centre's drift, the sample tiles' count, and the decision (every gate of the pass is on the
// device).
static int queue_bounds_gate(km_ctx *c, int k, const float *Cin, int64_t tstride, int nchunks, const int32_t *stop) {
    km_bnd *bs = c->bnd_st.p;
    HIPCHK(c, launch(c, KK_BOUNDS, [&] {
        return km_launch_bnd_drift(Cin, c->bnd_Clast.p, k, c->d, c->bnd_valid ? 1 : 0, c->bnd_S.p, c->bnd_delta.p, bs,
                                   stop, c->stream);
    }));
    const float hi = km_bnd_hi(c->d);
    int64_t row0 = 0;
    for (size_t i = 0; i < c->parts.size(); i++) {
        const Part &p = c->parts[i];
        HIPCHK(c, launch(c, KK_BOUNDS_SAMPLE, [&] {
            return km_launch_bnd_count(c->bnd_lb.p + c->bnd_off[i], c->bnd_ub.p + row0, c->bnd_ubl.p + row0, p.rows,
                                       k, nchunks, tstride, c->bnd_S.p, c->bnd_delta.p, hi, bs, stop, c->stream);
        }));
        row0 += p.rows;
    }
    HIPCHK(c, launch(c, KK_BOUNDS, [&] {
        return km_launch_bnd_decide(bs, c->bnd_max_visited, c->bnd_S.p, k, stop, c->stream);
    }));
    c->bnd_valid = true;
    return KM_OK;
}

// The wide-row pass: centre operands, then per slice the screen + exact rescoring (labels and best for every
// row), then per slice the sorted accumulation into one range sum per slice, then the finish. In the fit loop
// (lmode set) the labels alternate between two arrays by pass parity; a KM_LSTATE_DELTA pass counts the rows that
// changed since the previous pass and, when few did, accumulates only those (the full accumulation stands down).
static int run_big(km_ctx *c, int k, int mode, uint32_t *labels_d, float *best_d, const int32_t *stop, int pass,
                   double tol, int flags, int lmode) {
    const int d = c->d;
    const int64_t kw = (int64_t)k * (d + 2);
    const float *Cin = c->Cb[pass & 1].p;
    int64_t max_rows = 0;
    int max_nb = 0;
    bool built = false;
    for (auto &p : c->parts) {
        const km_big_plan bp = km_plan_big(p.rows, d, k);
        max_rows = std::max(max_rows, p.rows);
        max_nb = std::max(max_nb, bp.nb);
        if (!p.x16 || p.x16_ds != bp.DS) {
            built = true;
            if (p.x16) (void)hipFree(p.x16);
            if (p.xsq) (void)hipFree(p.xsq);
            p.x16 = nullptr;
            p.xsq = nullptr;
            HIPCHK(c, hipMalloc((void **)&p.x16, km_big_x16_elems(bp) * sizeof(uint16_t)));
            HIPCHK(c, hipMalloc((void **)&p.xsq, (size_t)p.rows * 2 * sizeof(float)));
            HIPCHK(c, launch(c, KK_BIG_PREP, [&] { return km_launch_big_rows(bp, p.X, p.rows, d, p.x16, p.xsq, c->stream); }));
            p.x16_ds = bp.DS;
        }
    }
    if (built) {   // a slice's row norms are new: the largest |x|^2 over all slices again
        HIPCHK(c, c->xmax.ensure(1));
        HIPCHK(c, hipMemsetAsync(c->xmax.p, 0, sizeof(uint32_t), c->stream));
        for (auto &p : c->parts)
            HIPCHK(c, launch(c, KK_BIG_PREP, [&] { return km_launch_big_xmax(p.xsq, p.rows, c->xmax.p, c->stream); }));
    }
    const km_big_plan bp0 = km_plan_big(max_rows, d, k);
    HIPCHK(c, c->cop.ensure(km_big_cop_elems(bp0)));
    HIPCHK(c, c->bcsq.ensure(bp0.kpad));
    HIPCHK(c, c->bcn.ensure((size_t)bp0.kpad * 2));
    HIPCHK(c, c->bmax.ensure(4));
    HIPCHK(c, c->ncand.ensure((size_t)max_rows));
    HIPCHK(c, c->cand.ensure((size_t)max_rows * 2 * km_big_list_slot(d)));
    HIPCHK(c, c->hist.ensure((size_t)max_nb * k));
    HIPCHK(c, c->counts.ensure((size_t)k));
    HIPCHK(c, c->base.ensure((size_t)k));
    HIPCHK(c, c->perm.ensure((size_t)max_rows));
    HIPCHK(c, c->over.ensure((size_t)max_rows));
    HIPCHK(c, c->multi.ensure((size_t)max_rows));
    HIPCHK(c, c->pieces.ensure((size_t)km_chunk_piece_doubles(max_rows, d, 0)));
    HIPCHK(c, c->okeys.ensure((size_t)max_rows));
    HIPCHK(c, c->labels.ensure((size_t)c->n));
    HIPCHK(c, c->best.ensure((size_t)c->n));
    HIPCHK(c, c->tot.ensure((size_t)kw));
    const int S = (int)c->parts.size();
    HIPCHK(c, c->red.ensure((size_t)S * kw));
    const bool wd = lmode != KM_LSTATE_NONE && !labels_d && !best_d;
    const bool delta = wd && lmode == KM_LSTATE_DELTA;
    if (wd) HIPCHK(c, c->wlab.ensure((size_t)c->n));
    uint32_t *lab_all = labels_d ? labels_d : (wd && (pass & 1)) ? c->wlab.p : c->labels.p;
    const uint32_t *lab_prev = (pass & 1) ? c->labels.p : c->wlab.p;
    float *best_all = best_d ? best_d : c->best.p;
    // without per-row outputs, single-candidate rows skip the rescoring and the accumulation adds the distances
    const int lite = (labels_d || best_d) ? 0 : 1;
    bool bnd = false;
    int64_t tstride = 1;
    {
        const int r = prepare_bounds(c, k, mode, bp0, &bnd, &tstride);
        if (r) return r;
    }
    km_bnd *bs = bnd ? c->bnd_st.p : nullptr;
    HIPCHK(c, launch(c, KK_BIG_PREP, [&] {
        return km_launch_big_centres(bp0, Cin, k, d, c->bcsq.p, c->bcn.p, c->cop.p, c->bmax.p, c->ctl, stop, c->stream);
    }));
    if (bnd) {
        const int r = queue_bounds_gate(c, k, Cin, tstride, bp0.nchunks, stop);
        if (r) return r;
    }
    int64_t row0 = 0;
    for (size_t i = 0; i < c->parts.size(); i++) {
        const Part &p = c->parts[i];
        const km_big_plan bp = km_plan_big(p.rows, d, k);
        if (i > 0)   // each slice lists its own overflow rows
            HIPCHK(c, launch(c, KK_BIG_PREP, [&] {
                return km_launch_big_centres(bp0, Cin, k, d, c->bcsq.p, c->bcn.p, c->cop.p, c->bmax.p, c->ctl, stop,
                                             c->stream);
            }));
        // a tracked pass: the plain screen, the building screen and the bounds list are all queued, and the
        // decision on the device lets the one this pass needs run
        float *sraw = bnd ? c->bnd_raw.p + c->bnd_soff[i] * bp.nchunks * 1024 : nullptr;
        HIPCHK(c, launch(c, KK_BIG_SCREEN, [&] {
            return km_launch_big_screen(bp, mode, p.x16, p.xsq, c->xmax.p, p.rows, d, c->cop.p, c->bmax.p, k,
                                        c->ncand.p, c->cand.p, c->over.p, c->multi.p, c->ctl,
                                        bnd ? &bs->skip_plain : stop, c->stream, sraw, tstride);
        }));
        km_bnd_refresh bref{};
        if (bnd) {
            uint16_t *lb = c->bnd_lb.p + c->bnd_off[i];
            bref = km_bnd_refresh{lb, c->bnd_ub.p + row0, c->bnd_ubl.p + row0, c->bnd_S.p, bp.nchunks,
                                  km_bnd_lo(d) * (1.0f - 0x1p-21f), km_bnd_hi(d) * (1.0f + 0x1p-21f), bs};
            HIPCHK(c, launch(c, KK_BOUNDS_SAMPLE, [&] {
                return km_launch_bnd_resample(sraw, p.xsq, p.rows, d, bp.DS, c->bmax.p, k, bp.nchunks, tstride, lb,
                                              bref.ub, bref.ubl, c->bnd_S.p, bs, c->stream);
            }));
            HIPCHK(c, launch(c, KK_BIG_SCREEN_BND, [&] {
                return km_launch_big_screen_bnd(bp, p.x16, p.xsq, p.rows, d, c->cop.p, c->bmax.p, k, c->ncand.p,
                                                c->cand.p, c->over.p, c->multi.p, c->ctl, lb, bref.ub, bref.ubl, bs,
                                                c->dev.cus, c->stream);
            }));
            HIPCHK(c, launch(c, KK_BOUNDS_LIST, [&] {
                return km_launch_bnd_list(lb, bref.ub, bref.ubl, p.rows, k, bp.nchunks, c->bnd_S.p, c->bnd_delta.p,
                                          km_bnd_hi(d), c->ncand.p, c->cand.p, km_big_list_slot(d), c->over.p,
                                          c->multi.p, c->ctl, bs, c->dev.cus, c->stream);
            }));
        }
        HIPCHK(c, launch(c, KK_BIG_RESCORE, [&] {
            return km_launch_big_rescore(p.X, p.rows, d, Cin, k, c->ncand.p, c->cand.p, c->over.p, c->multi.p,
                                         c->ctl, lab_all + row0, best_all + row0, lite, c->okeys.p, stop, c->stream,
                                         bnd ? &bref : nullptr);
        }));
        row0 += p.rows;
    }
    const int32_t *full_gate = stop;
    if (delta) {   // the gate: the change-only sums or the full accumulation, chosen on the device
        HIPCHK(c, launch(c, KK_CHANGE, [&] {
            return km_launch_wd_gate(lab_all, lab_prev, c->n, c->wd_limit, c->wd_bcnt.p, c->wd_gate.p, stop, c->stream);
        }));
        full_gate = c->wd_gate.p + 1;
    }
    row0 = 0;
    for (size_t i = 0; i < c->parts.size(); i++) {
        const Part &p = c->parts[i];
        const km_big_plan bp = km_plan_big(p.rows, d, k);
        HIPCHK(c, launch(c, KK_BIG_ACCUM, [&] {
            return km_launch_big_accum(bp, p.X, p.rows, d, lab_all + row0, best_all + row0, lite ? Cin : nullptr, k,
                                       c->hist.p, c->counts.p, c->base.p, c->perm.p, c->pieces.p,
                                       c->red.p + (int64_t)i * kw, full_gate, c->stream);
        }));
        row0 += p.rows;
    }
    if (!delta) return finish_pass(c, k, 0, pass, tol, flags, stop, S);
    HIPCHK(c, launch(c, KK_CHANGE, [&] {
        return km_launch_wd_accum(c->wd_slices.p, (int)c->parts.size(), c->n, d, lab_all, lab_prev, k, c->wd_limit,
                                  c->wd_bcnt.p, c->wd_e.p, c->wd_e.p + 2 * c->wd_limit, c->wd_H.p, c->wd_cnt.p,
                                  c->wd_base.p, c->wd_perm.p, c->pieces.p, c->red.p, c->wd_gate.p, c->stream);
    }));
    return finish_pass(c, k, 0, pass, tol, flags, stop, S, c->wd_gate.p);
}

// Pass `pass`: assignment + accumulation over every slice with the centres in Cb[pass & 1], then the finish
// (float64 totals in c->tot; with KM_FIN_UPDATE in flags the new centres and the statistics). labels_d/best_d:
// device arrays of n (or null) for the per-row results. gated: every kernel checks ctl->stop first.
static int run_pass(km_ctx *c, int k, int mode, int path, uint32_t *labels_d, float *best_d, bool gated, int pass,
                    double tol, int flags, int lmode = KM_LSTATE_NONE) {
    HIPCHK(c, c->Cb[(pass + 1) & 1].ensure((size_t)k * c->d));
    const float *Cin = c->Cb[pass & 1].p;
    km_mfma_plan mp;
    const int fam = choose_path(c, k, path, &mp);
    if (fam < 0)
        return fail(c, KM_EINVAL, "path=%s does not serve k=%d, dims=%d on this build",
                    path == KM_PATH_MFMA ? "mfma" : "fused", k, c->d);
    c->last_path = family_path(fam);
    c->last_family = fam;
    const int32_t *stop = gated ? &c->ctl->stop : nullptr;
    const int d = c->d;

    if (fam == FAM_BIG) return run_big(c, k, mode, labels_d, best_d, stop, pass, tol, flags, lmode);

    if (fam == FAM_MFMA_FUSED) {
        // without per-row outputs the kernel skips the direct form for rows the screen settles alone
        const int want_best = (labels_d || best_d) ? 1 : 0;
        size_t total_rb = 0;
        std::vector<km_mfma_plan> plans;
        for (auto &p : c->parts) {
            plans.push_back(km_plan_mfma(c->dev, p.rows, d, k));
            total_rb += plans.back().nrb;
        }
        int r = ensure_pass_buffers(c, k, total_rb, false);
        if (r) return r;
        // a change-only pass writes only the rows of partials its changed rows touched, and says which
        uint32_t *pm = nullptr;
        if (lmode == KM_LSTATE_DELTA) {
            HIPCHK(c, c->pmask.ensure(total_rb * KM_PMASK_WORDS));
            pm = c->pmask.p;
        }
        // where the last fit saw few open rows, its change-only passes take the kernel without candidate lists
        const int scan_only = lmode == KM_LSTATE_DELTA && c->open_frac >= 0.0 && c->open_frac <= KM_SCAN_ONLY_FRAC;
        int rb = 0;
        int64_t row0 = 0;
        for (size_t i = 0; i < c->parts.size(); i++) {
            const Part &p = c->parts[i];
            uint32_t *lab = labels_d ? labels_d + row0 : nullptr;
            float *bst = best_d ? best_d + row0 : nullptr;
            uint8_t *ls = lmode != KM_LSTATE_NONE ? c->lstate.p + c->lstate_off[i] : nullptr;
            HIPCHK(c, launch(c, KK_FUSED_MFMA, [&] {
                return km_launch_mfma(plans[i], want_best, p.X, p.rows, d, Cin, k, lab, bst, c->psum.p, c->pcomp.p,
                                      rb, c->ctl, ls, ls, lmode, stop, c->stream, scan_only, pm);
            }));
            rb += plans[i].nrb;
            row0 += p.rows;
        }
        return finish_pass(c, k, rb, pass, tol, flags | (lmode == KM_LSTATE_DELTA ? KM_FIN_DELTA : 0), stop, 0,
                           nullptr, pm);
    }

    if (fam == FAM_LOWD) {
        size_t total_rb = 0;
        std::vector<km_lowd_plan> plans;
        const bool al = parts_aligned(c);
        for (auto &p : c->parts) {
            plans.push_back(km_plan_lowd(c->dev, p.rows, d, k, al));
            total_rb += plans.back().nrb;
        }
        int r = ensure_pass_buffers(c, k, total_rb, false);
        if (r) return r;
        int rb = 0;
        int64_t row0 = 0;
        for (size_t i = 0; i < c->parts.size(); i++) {
            const Part &p = c->parts[i];
            uint32_t *lab = labels_d ? labels_d + row0 : nullptr;
            float *bst = best_d ? best_d + row0 : nullptr;
            HIPCHK(c, launch(c, KK_FUSED_LOWD, [&] {
                return km_launch_lowd(plans[i], p.X, p.rows, d, Cin, k, lab, bst, c->psum.p, c->pcomp.p, rb, stop,
                                      c->stream);
            }));
            rb += plans[i].nrb;
            row0 += p.rows;
        }
        return finish_pass(c, k, rb, pass, tol, flags, stop);
    }

    // rows path: exact labels for every slice, then the generic accumulation (or, at large k, the counting sort)
    if (k > KM_SORTED_MIN_K) {
        const int64_t kw = (int64_t)k * (d + 2);
        int64_t max_rows = 0;
        for (auto &p : c->parts) max_rows = std::max(max_rows, p.rows);
        HIPCHK(c, c->labels.ensure((size_t)c->n));
        HIPCHK(c, c->best.ensure((size_t)c->n));
        HIPCHK(c, c->hist.ensure((size_t)km_sorted_blocks(max_rows) * k));
        HIPCHK(c, c->counts.ensure((size_t)k));
        HIPCHK(c, c->base.ensure((size_t)k));
        HIPCHK(c, c->perm.ensure((size_t)max_rows));
        HIPCHK(c, c->pieces.ensure((size_t)km_chunk_piece_doubles(max_rows, d, 0)));
        HIPCHK(c, c->tot.ensure((size_t)kw));
        const int S = (int)c->parts.size();
        HIPCHK(c, c->red.ensure((size_t)S * kw));
        uint32_t *lab_all = labels_d ? labels_d : c->labels.p;
        float *best_all = best_d ? best_d : c->best.p;
        int64_t row0 = 0;
        for (size_t i = 0; i < c->parts.size(); i++) {
            const Part &p = c->parts[i];
            HIPCHK(c, launch(c, KK_ASSIGN_ROWS, [&] {
                return km_launch_assign_rows(p.X, p.rows, d, Cin, k, lab_all + row0, best_all + row0, stop, c->stream);
            }));
            HIPCHK(c, launch(c, KK_ACCUM_GENERIC, [&] {
                return km_launch_sorted_accum(p.X, p.rows, d, lab_all + row0, best_all + row0, k, c->hist.p,
                                              c->counts.p, c->base.p, c->perm.p, c->pieces.p,
                                              c->red.p + (int64_t)i * kw, stop, c->stream);
            }));
            row0 += p.rows;
        }
        return finish_pass(c, k, 0, pass, tol, flags, stop, S);
    }
    size_t total_rb = 0;
    std::vector<km_accum_plan> plans;
    for (auto &p : c->parts) {
        plans.push_back(km_plan_accum_generic(p.rows, d, k));
        total_rb += plans.back().nrb;
    }
    int r = ensure_pass_buffers(c, k, total_rb, true);
    if (r) return r;
    uint32_t *lab_all = labels_d ? labels_d : c->labels.p;
    float *best_all = best_d ? best_d : c->best.p;
    int rb = 0;
    int64_t row0 = 0;
    for (size_t i = 0; i < c->parts.size(); i++) {
        const Part &p = c->parts[i];
        HIPCHK(c, launch(c, KK_ASSIGN_ROWS, [&] {
            return km_launch_assign_rows(p.X, p.rows, d, Cin, k, lab_all + row0, best_all + row0, stop, c->stream);
        }));
        HIPCHK(c, launch(c, KK_ACCUM_GENERIC, [&] {
            return km_launch_accum_generic(plans[i], p.X, p.rows, d, lab_all + row0, best_all + row0, k, c->psum.p,
                                           c->pcomp.p, rb, stop, c->stream);
        }));
        rb += plans[i].nrb;
        row0 += p.rows;
    }
    return finish_pass(c, k, rb, pass, tol, flags, stop);
}

// Labels and best for every row with the centres in Cb[pass & 1], into c->labels / c->best. The pass runs in
// full (it is the same code as every other pass, so the same bits) but updates nothing.
static int run_labels(km_ctx *c, int k, int mode, int path, int pass) {
    HIPCHK(c, c->labels.ensure((size_t)c->n));
    HIPCHK(c, c->best.ensure((size_t)c->n));
    return run_pass(c, k, mode, path, c->labels.p, c->best.p, false, pass, 0.0, 0);
}

static int upload_centres(km_ctx *c, const float *C, int k) {
    HIPCHK(c, c->Cb[0].ensure((size_t)k * c->d));
    HIPCHK(c, c->Cb[1].ensure((size_t)k * c->d));
    HIPCHK(c, hipMemcpyAsync(c->Cb[0].p, C, (size_t)k * c->d * sizeof(float), hipMemcpyHostToDevice, c->stream));
    return KM_OK;
}

// The host mirror is pinned: the copy reads it when the stream reaches it, and nothing writes the mirror before the
// next read_control (a copy into it, ordered after this one) or a synchronisation, so the caller queues its passes
// without waiting here.
static int reset_control(km_ctx *c, double tol) {
    HIPCHK(c, hipStreamSynchronize(c->stream));   // no copy into the mirror is still in flight
    memset(c->ctl_h, 0, sizeof(km_control));
    c->ctl_h->tol = tol;
    HIPCHK(c, hipMemcpyAsync(c->ctl, c->ctl_h, sizeof(km_control), hipMemcpyHostToDevice, c->stream));
    return KM_OK;
}

static int read_control(km_ctx *c) {
    HIPCHK(c, hipMemcpyAsync(c->ctl_h, c->ctl, sizeof(km_control), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KM_OK;
}

static int write_control(km_ctx *c) {
    HIPCHK(c, hipMemcpyAsync(c->ctl, c->ctl_h, sizeof(km_control), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return KM_OK;
}

extern "C" int32_t km_pass(km_ctx *c, const float *C, int32_t k, int32_t mode, int32_t path, double *totals,
                           uint32_t *labels, float *best) {
    if (!c) return KM_EINVAL;
    int r = check_centres(c, C, k);
    if (r) return r;
    if (!totals) return fail(c, KM_EINVAL, "totals pointer is null");
    HIPCHK(c, hipSetDevice(c->device));
    if ((r = upload_centres(c, C, k))) return r;
    HIPCHK(c, c->labels.ensure((size_t)c->n));
    HIPCHK(c, c->best.ensure((size_t)c->n));
    if ((r = reset_control(c, 0.0))) return r;
    if ((r = run_pass(c, k, mode, path, c->labels.p, c->best.p, false, 0, 0.0, 0))) return r;
    const int w = c->d + 2;
    const int64_t kw = (int64_t)k * w;
    HIPCHK(c, hipMemcpyAsync(totals, c->tot.p, kw * sizeof(double), hipMemcpyDeviceToHost, c->stream));
    std::vector<double> cb2;
    if (c->last_family == FAM_MFMA_FUSED) {
        // The fused screen keeps the per-cluster sums of x but only the pass total of best (column 1 of
        // cluster 0). The per-cluster best sums come from one more deterministic accumulation over the
        // [count, best] columns alone, reading the labels and best this pass wrote.
        std::vector<km_accum_plan> plans;
        size_t total_rb = 0;
        for (auto &p : c->parts) {
            plans.push_back(km_plan_accum_generic(p.rows, 0, k));
            total_rb += plans.back().nrb;
        }
        HIPCHK(c, c->psum.ensure(total_rb * (size_t)k * 2));
        HIPCHK(c, c->pcomp.ensure(total_rb * (size_t)k * 2));
        HIPCHK(c, c->tot2.ensure((size_t)k * 2));
        const int S2 = km_reduce_splits((int)total_rb, (int64_t)k * 2, c->dev.cus);
        HIPCHK(c, c->red.ensure((size_t)S2 * k * 2));
        int rb = 0;
        int64_t row0 = 0;
        for (size_t i = 0; i < c->parts.size(); i++) {
            const Part &p = c->parts[i];
            HIPCHK(c, launch(c, KK_ACCUM_GENERIC, [&] {
                return km_launch_accum_generic(plans[i], nullptr, p.rows, 0, c->labels.p + row0, c->best.p + row0, k,
                                               c->psum.p, c->pcomp.p, rb, nullptr, c->stream);
            }));
            rb += plans[i].nrb;
            row0 += p.rows;
        }
        HIPCHK(c, launch(c, KK_REDUCE, [&] {
            return km_launch_reduce_finish(c->psum.p, c->pcomp.p, rb, (int64_t)k * 2, S2, c->red.p, k, 0, c->tot2.p,
                                           nullptr, c->ctl, 0, 0.0, 0, nullptr, c->stream);
        }));
        cb2.resize((size_t)k * 2);
        HIPCHK(c, hipMemcpyAsync(cb2.data(), c->tot2.p, cb2.size() * sizeof(double), hipMemcpyDeviceToHost, c->stream));
    }
    if (labels) HIPCHK(c, hipMemcpyAsync(labels, c->labels.p, c->n * sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream));
    if (best) HIPCHK(c, hipMemcpyAsync(best, c->best.p, c->n * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (!cb2.empty())
        for (int j = 0; j < k; j++) totals[(size_t)j * w + 1] = cb2[(size_t)j * 2 + 1];
    harvest(c);
    return KM_OK;
}

// ------------------------------------------------------------------ relocation of empty clusters
//
// The pass `pass` whose statistics flagged empties left its totals in c->tot and its input centres in
// Cb[pass & 1]; the relocated centres go to Cb[(pass + 1) & 1].
// Following lloyd_step (core.py:2222-2242): the empty clusters, in ascending order, take the rows with the
// largest best distance (ties: lower row index); each such row leaves its old cluster; centres are the
// float64 means rounded to float32; a cluster still empty takes the largest cluster's centre. All of it runs on
// the device (km_reloc.hip): the host reads back only the number of empty clusters.
static int relocate(km_ctx *c, int k, int mode, int path, int pass, int *n_empty_out) {
    const int d = c->d;
    int r = run_labels(c, k, mode, path, pass);
    if (r) return r;
    const int64_t nb = km_reloc_blocks(c->n, c->dev.cus);
    HIPCHK(c, c->rl_st.ensure(km_reloc_state_words()));
    HIPCHK(c, c->rl_empty.ensure((size_t)k));
    HIPCHK(c, c->rl_sel.ensure(2 * (size_t)k));
    HIPCHK(c, c->rl_tie.ensure((size_t)nb));
    HIPCHK(c, c->rl_ws.ensure((size_t)k * (d + 2)));
    HIPCHK(c, c->rl_parts.ensure(c->parts.size() * 16));
    std::vector<const float *> px;
    std::vector<int64_t> pr;
    for (auto &p : c->parts) {
        px.push_back(p.X);
        pr.push_back(p.rows);
    }
    HIPCHK(c, launch(c, KK_RELOCATE, [&] {
        return km_launch_relocate(c->tot.p, k, d, c->n, c->best.p, c->labels.p, px.data(), pr.data(), (int)px.size(),
                                  c->rl_parts.p, c->rl_st.p, c->rl_empty.p, c->rl_sel.p, c->rl_sel.p + k, c->rl_tie.p,
                                  c->rl_ws.p, c->Cb[(pass + 1) & 1].p, c->dev.cus, c->stream);
    }));
    uint32_t ne = 0;
    HIPCHK(c, hipMemcpyAsync(&ne, c->rl_st.p + KM_RELOC_NEMPTY_WORD, sizeof ne, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *n_empty_out = (int)ne;
    return KM_OK;
}

// Queues pass `pass` of a loop, gated on the control block.
static int queue_iteration(km_ctx *c, int k, int mode, int path, int pass, double tol, int spherical,
                           int lmode = KM_LSTATE_NONE) {
    return run_pass(c, k, mode, path, nullptr, nullptr, true, pass, tol,
                    KM_FIN_UPDATE | (spherical ? KM_FIN_SPHERICAL : 0), lmode);
}

// The most changed rows a pass of the wide-row path takes as change-only sums: they sort 2m entries and read each
// changed row twice, the full accumulation sorts and reads every row once; below half the rows the change-only
// sums are the cheaper.
static int64_t wide_delta_limit(int64_t n) { return n / 2; }

// The wide-row path's change-only accumulation: the second label array, the count and entry arrays, and once per
// data set the slice table and [mu, T] (queued on the stream before the loop's first pass).
static int prepare_wide_delta(km_ctx *c, int k, bool *use) {
    *use = false;
    const int d = c->d;
    if (d > km_wd_max_dims() || c->n > (int64_t)0x7fffffff) return KM_OK;
    const int64_t limit = wide_delta_limit(c->n);
    if (limit < 1) return KM_OK;
    c->wd_limit = limit;
    HIPCHK(c, c->labels.ensure((size_t)c->n));
    HIPCHK(c, c->wlab.ensure((size_t)c->n));
    HIPCHK(c, c->wd_bcnt.ensure((size_t)km_wd_blocks(c->n) + 1));
    HIPCHK(c, c->wd_e.ensure((size_t)limit * 4));
    HIPCHK(c, c->wd_H.ensure((size_t)km_sorted_blocks(2 * limit) * k));
    HIPCHK(c, c->wd_cnt.ensure((size_t)k));
    HIPCHK(c, c->wd_base.ensure((size_t)k));
    HIPCHK(c, c->wd_perm.ensure((size_t)limit * 2));
    int64_t max_rows = 0;
    for (auto &p : c->parts) max_rows = std::max(max_rows, p.rows);
    HIPCHK(c, c->pieces.ensure((size_t)std::max(km_chunk_piece_doubles(2 * limit, d, 2),
                                                 km_chunk_piece_doubles(max_rows, d, 0))));
    HIPCHK(c, c->wd_gate.ensure(2));
    if (!c->wd_ready) {
        std::vector<int64_t> rows;
        int64_t nb = 0, row0 = 0;
        c->wd_slices_h.clear();
        for (auto &p : c->parts) {
            c->wd_slices_h.push_back({p.X, row0});
            rows.push_back(p.rows);
            nb += km_wd_stat_blocks(p.rows);
            row0 += p.rows;
        }
        HIPCHK(c, c->wd_part.ensure((size_t)nb * (d + 1)));
        HIPCHK(c, c->wd_mu.ensure((size_t)d + 1));
        HIPCHK(c, c->wd_slices.ensure(c->wd_slices_h.size()));
        HIPCHK(c, hipMemcpyAsync(c->wd_slices.p, c->wd_slices_h.data(), c->wd_slices_h.size() * sizeof(km_slice),
                                 hipMemcpyHostToDevice, c->stream));
        HIPCHK(c, launch(c, KK_BIG_PREP, [&] {
            return km_launch_wd_stats(c->wd_slices_h.data(), rows.data(), (int)rows.size(), d, c->wd_part.p,
                                      c->wd_mu.p, c->stream);
        }));
        c->wd_ready = true;
    }
    *use = true;
    return KM_OK;
}

// The fit loop keeps every row's label between passes where the fused MFMA path or the wide-row path runs, so
// that a pass accumulates only the rows whose label changed. For the fused MFMA path: sizes the label array (each
// slice's at a 64-row-aligned offset, 64 bytes of padding after it). Returns whether the loop uses it.
static int prepare_label_state(km_ctx *c, int k, bool *use) {
    km_mfma_plan mp;
    const int fam = choose_path(c, k, KM_PATH_AUTO, &mp);
    if (fam == FAM_BIG) return prepare_wide_delta(c, k, use);
    *use = fam == FAM_MFMA_FUSED && k <= 256;
    if (!*use) return KM_OK;
    c->lstate_off.clear();
    int64_t off = 0;
    for (auto &p : c->parts) {
        c->lstate_off.push_back(off);
        off += (p.rows + 64 + 63) / 64 * 64;
    }
    HIPCHK(c, c->lstate.ensure((size_t)off));
    return KM_OK;
}

extern "C" int32_t km_lloyd_step(km_ctx *c, const float *C, int32_t k, int32_t mode, int32_t path, float *C_out,
                                 double *inertia, int32_t *n_empty) {
    if (!c) return KM_EINVAL;
    int r = check_centres(c, C, k);
    if (r) return r;
    if (!C_out) return fail(c, KM_EINVAL, "C_out pointer is null");
    HIPCHK(c, hipSetDevice(c->device));
    if ((r = upload_centres(c, C, k))) return r;
    if ((r = reset_control(c, 0.0))) return r;
    if ((r = queue_iteration(c, k, mode, path, 0, 0.0, 0))) return r;
    if ((r = read_control(c))) return r;
    int ne = c->ctl_h->n_empty;
    if (c->ctl_h->need_reloc) {
        if ((r = relocate(c, k, mode, path, 0, &ne))) return r;
    }
    HIPCHK(c, hipMemcpyAsync(C_out, c->Cb[1].p, (size_t)k * c->d * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (inertia) *inertia = c->ctl_h->inertia;
    if (n_empty) *n_empty = ne;
    harvest(c);
    return KM_OK;
}

extern "C" int32_t km_fit(km_ctx *c, const float *C0, int32_t k, int32_t max_iter, double tol, int32_t mode,
                          int32_t spherical, float *C_out, double *last_inertia, int32_t *n_iter,
                          int32_t *n_relocated) {
    if (!c) return KM_EINVAL;
    int r = check_centres(c, C0, k);
    if (r) return r;
    if (max_iter < 1) return fail(c, KM_EINVAL, "max_iter must be a positive integer");
    if (std::isnan(tol)) return fail(c, KM_EINVAL, "tol must not be NaN");
    HIPCHK(c, hipSetDevice(c->device));
    if ((r = upload_centres(c, C0, k))) return r;
    if ((r = reset_control(c, tol))) return r;
    if (spherical) HIPCHK(c, launch(c, KK_NORMALISE, [&] { return km_launch_normalise(c->Cb[0].p, k, c->d, c->stream); }));
    const int path = KM_PATH_AUTO;
    bool use_ls = false;
    if ((r = prepare_label_state(c, k, &use_ls))) return r;
    // the pass that records every label (the first, and the first after a relocation); later passes accumulate
    // only the rows whose label changed, and every KM_REANCHOR_PASSES-th pass after it records again
    int rec_pass = 0;
    int pass = 0, relocated = 0;
    // with timing on, an event at every pass boundary on the stream: the per-pass times km_profile_passes reads
    std::vector<std::vector<hipEvent_t>> marks;   // per batch: one before each pass, one after the last
    auto mark = [&](bool first) {
        if (!c->prof) return;
        if (first) marks.emplace_back();
        hipEvent_t e = get_event(c);
        if (e && hipEventRecord(e, c->stream) == hipSuccess) marks.back().push_back(e);
    };
    while (pass < max_iter) {
        const int batch = std::min(KM_FIT_BATCH, max_iter - pass);
        for (int i = 0; i < batch; i++) {
            const int since = pass + i - rec_pass;
            const int lm = !use_ls ? KM_LSTATE_NONE
                                   : (since % KM_REANCHOR_PASSES == 0 ? KM_LSTATE_RECORD : KM_LSTATE_DELTA);
            mark(i == 0);
            if ((r = queue_iteration(c, k, mode, path, pass + i, tol, spherical, lm))) return r;
        }
        mark(false);
        if ((r = read_control(c))) return r;
        pass = c->ctl_h->iter;
        if (c->last_family == FAM_MFMA_FUSED && pass > 0)
            c->open_frac = (double)c->ctl_h->fallback_rows / ((double)c->n * pass);
        if (c->ctl_h->need_reloc) {
            int ne = 0;
            const int q = c->ctl_h->iter - 1;   // the pass that left clusters empty
            if ((r = relocate(c, k, mode, path, q, &ne))) return r;
            relocated += ne;
            rec_pass = q + 1;   // relocation moved rows and totals: the next pass starts the label state again
            if (spherical)
                HIPCHK(c, launch(c, KK_NORMALISE, [&] { return km_launch_normalise(c->Cb[(q + 1) & 1].p, k, c->d, c->stream); }));
            c->ctl_h->need_reloc = 0;
            c->ctl_h->stop = c->ctl_h->done;
            if ((r = write_control(c))) return r;
        }
        if (c->ctl_h->done || !std::isfinite(c->ctl_h->inertia)) break;
    }
    if (C_out)
        HIPCHK(c, hipMemcpyAsync(C_out, c->Cb[c->ctl_h->iter & 1].p, (size_t)k * c->d * sizeof(float),
                                 hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (last_inertia) *last_inertia = c->ctl_h->inertia;
    if (n_iter) *n_iter = c->ctl_h->iter;
    if (n_relocated) *n_relocated = relocated;
    // within a batch consecutive marks bracket one pass (between batches the host reads the control block)
    for (auto &b : marks) {
        for (size_t i = 0; i + 1 < b.size(); i++) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, b[i], b[i + 1]) == hipSuccess) c->pass_ms.push_back(ms);
        }
        for (auto e : b) c->pool.push_back(e);
    }
    harvest(c);
    return KM_OK;
}

// ------------------------------------------------------------------ k-means++ seeding

extern "C" int32_t km_seed_pp(km_ctx *c, int32_t k, const int64_t *sample, int64_t m, int64_t first,
                              const uint64_t *seeds, float *C_out) {
    if (!c) return KM_EINVAL;
    if (c->n == 0) return fail(c, KM_ENODATA, "no data set on the context");
    if (k < 1) return fail(c, KM_EINVAL, "n_clusters must be a positive integer");
    if (!sample || !C_out || (k > 1 && !seeds)) return fail(c, KM_EINVAL, "sample, seeds and C_out must not be null");
    if (m < k) return fail(c, KM_EINVAL, "n_samples=%lld should be >= n_clusters=%d", (long long)m, k);
    if (m > (int64_t)UINT32_MAX) return fail(c, KM_EINVAL, "a sample of %lld rows exceeds 32-bit row indices", (long long)m);
    if (first < 0 || first >= m) return fail(c, KM_EINVAL, "first pick %lld is outside the sample", (long long)first);
    if (km_pp_trials(k) > KM_PP_MAX_TRIALS) return fail(c, KM_EINVAL, "n_clusters=%d is too large for k-means++ seeding", k);
    for (int64_t j = 0; j < m; j++)
        if (sample[j] < 0 || sample[j] >= c->n || (j > 0 && sample[j] < sample[j - 1]))
            return fail(c, KM_EINVAL, "sample rows must be ascending row indices below %lld", (long long)c->n);
    HIPCHK(c, hipSetDevice(c->device));
    const int d = c->d;
    HIPCHK(c, c->pp_S.ensure((size_t)m * d));
    HIPCHK(c, c->pp_R.ensure((size_t)m * d));
    HIPCHK(c, c->pp_C.ensure((size_t)k * d));
    HIPCHK(c, c->pp_idx.ensure((size_t)m));
    HIPCHK(c, c->pp_ws.ensure(km_pp_workspace(m, k)));
    // the sample's rows, slice by slice (the indices are ascending, so each slice takes one contiguous range)
    std::vector<int64_t> local(sample, sample + m);
    std::vector<int64_t> j0s, j1s;
    int64_t off = 0, j = 0;
    for (auto &p : c->parts) {
        const int64_t a = j;
        while (j < m && sample[j] < off + p.rows) {
            local[j] -= off;
            j++;
        }
        j0s.push_back(a);
        j1s.push_back(j);
        off += p.rows;
    }
    HIPCHK(c, hipMemcpyAsync(c->pp_idx.p, local.data(), (size_t)m * sizeof(int64_t), hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, launch(c, KK_SEED_PP, [&] {
        for (size_t q = 0; q < c->parts.size(); q++) {
            hipError_t e = km_launch_pp_gather(c->parts[q].X, c->pp_idx.p, j0s[q], j1s[q], m, d, c->pp_S.p, c->pp_R.p,
                                               c->stream);
            if (e != hipSuccess) return e;
        }
        return km_launch_pp(c->pp_S.p, c->pp_R.p, m, d, k, first, seeds, c->pp_ws.p, c->pp_C.p, c->stream);
    }));
    HIPCHK(c, hipMemcpyAsync(C_out, c->pp_C.p, (size_t)k * d * sizeof(float), hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    harvest(c);
    return KM_OK;
}

// ------------------------------------------------------------------ one pass without allocation
//
// The pass of km_pass for device rows and device centres, with every workspace carved out of the context's
// scratch (a control block, per-block partials, range sums) and the results written to the caller's device
// buffers, all on the caller's stream: no allocation, no host copy, no synchronisation. The exact kernel families
// of km_pass serve it, except the wide-row path (its bf16 copy of the rows is as large as the data): shapes it
// would take run the rows path, whose labels and best are the same bits.

// Zero n words (a kernel, not hipMemsetAsync: a caller may capture the stream into a graph).
__global__ __launch_bounds__(256) void k_na_clear(uint32_t *__restrict__ p, int n) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) p[i] = 0u;
}

// totals[c][1] = tot2[c][1]: the per-cluster best sums of the [count, best] accumulation.
__global__ __launch_bounds__(256) void k_na_best_col(const double *__restrict__ tot2, int k, int w,
                                                     double *__restrict__ totals) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < k) totals[(int64_t)c * w + 1] = tot2[(int64_t)c * 2 + 1];
}

// Bump allocator over the scratch array: 256-byte aligned pieces, false once it is exhausted.
struct ScratchCarve {
    unsigned char *base;
    size_t used, cap;
    template <class T>
    bool take(T **p, size_t count) {
        const size_t bytes = (count * sizeof(T) + 255) / 256 * 256;
        if (used + bytes > cap) return false;
        *p = reinterpret_cast<T *>(base + used);
        used += bytes;
        return true;
    }
};

// Bytes of scratch the reduce + finish of nrb partials of kw entries use (partials included).
static size_t na_reduce_bytes(int nrb, int64_t kw) {
    const int S = km_reduce_splits(nrb, kw, 1 << 30);   // the most range sums any device's split takes
    auto r = [](size_t b) { return (b + 255) / 256 * 256; };
    return 2 * r((size_t)nrb * kw * sizeof(float)) + r((size_t)S * kw * sizeof(double));
}

// Largest block count whose partials + range sums fit `avail` bytes (at least 1, or 0 if even one does not).
static int64_t na_max_blocks(size_t avail, int64_t kw) {
    int64_t lo = 0, hi = 1 << 20;
    while (lo < hi) {   // largest nrb with na_reduce_bytes(nrb) <= avail
        const int64_t mid = (lo + hi + 1) / 2;
        if (na_reduce_bytes((int)mid, kw) <= avail) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

extern "C" int32_t km_pass_noalloc(km_ctx *c, const float *X, int64_t rows, int32_t dims, const float *C, int32_t k,
                                   double *totals, uint32_t *labels, float *best, void *stream) {
    if (!c) return KM_EINVAL;
    if (!X || !C || !totals || !labels || !best)
        return fail(c, KM_EINVAL, "km_pass_noalloc: rows, centres, totals, labels and best must all be device pointers");
    if (rows < 1 || dims < 1) return fail(c, KM_EINVAL, "expected a nonempty 2-D (rows, dims) array, got %lld x %d",
                                          (long long)rows, dims);
    if (k < 1) return fail(c, KM_EINVAL, "n_clusters must be a positive integer");
    if (!c->scratch) return fail(c, KM_EDEVICE, "km_pass_noalloc: the scratch array's device address is unknown");
    const int d = dims;
    const int64_t kw = (int64_t)k * (d + 2);
    hipStream_t s = (hipStream_t)stream;
    HIPCHK(c, hipSetDevice(c->device));
    const bool al = ((uintptr_t)X % 16) == 0;
    ScratchCarve sc{c->scratch, 0, KM_SCRATCH_BYTES};
    km_control *ctl = nullptr;
    sc.take(&ctl, 1);
    // the family km_pass would run, the wide-row path excepted
    km_mfma_plan mp = km_plan_mfma(c->dev, rows, d, k);
    if (!al) mp.ok = 0;
    int fam;
    if (mp.ok && d >= 16 && (int64_t)k * d >= 192) fam = FAM_MFMA_FUSED;
    else if (km_plan_lowd(c->dev, rows, d, k, al).ok) fam = FAM_LOWD;
    else fam = FAM_ROWS;
    // the fused MFMA pass also accumulates [count, best] from its labels for the per-cluster best sums
    const int64_t kw2 = (int64_t)k * 2;
    km_accum_plan p2{};
    size_t extra = 0;
    if (fam == FAM_MFMA_FUSED) {
        const size_t avail2 = KM_SCRATCH_BYTES / 8;
        p2 = km_plan_accum_generic(rows, 0, k, na_max_blocks(avail2, kw2));
        extra = na_reduce_bytes(p2.nrb, kw2) + ((size_t)kw2 * sizeof(double) + 255) / 256 * 256;
        if (extra > avail2)
            return fail(c, KM_EINVAL, "km_pass_noalloc: k = %d needs more than the %zu bytes of scratch", k,
                        (size_t)KM_SCRATCH_BYTES);
    }
    const size_t avail = KM_SCRATCH_BYTES - sc.used - extra;
    const int64_t maxb = na_max_blocks(avail, kw);
    if (maxb < 1)
        return fail(c, KM_EINVAL, "km_pass_noalloc: k * (dims + 2) = %lld entries need more than the %zu bytes of "
                    "scratch (one block's partials and range sums); use km_pass", (long long)kw,
                    (size_t)KM_SCRATCH_BYTES);
    int nrb;
    km_lowd_plan lp{};
    km_accum_plan ap{};
    if (fam == FAM_MFMA_FUSED) {
        mp = km_plan_mfma(c->dev, rows, d, k, maxb);
        nrb = mp.nrb;
    } else if (fam == FAM_LOWD) {
        lp = km_plan_lowd(c->dev, rows, d, k, al, maxb);
        nrb = lp.nrb;
    } else {
        ap = km_plan_accum_generic(rows, d, k, maxb);
        nrb = ap.nrb;
    }
    const int S = km_reduce_splits(nrb, kw, c->dev.cus);
    float *psum = nullptr, *pcomp = nullptr;
    double *red = nullptr;
    if (!sc.take(&psum, (size_t)nrb * kw) || !sc.take(&pcomp, (size_t)nrb * kw) || !sc.take(&red, (size_t)S * kw))
        return fail(c, KM_EINVAL, "km_pass_noalloc: the pass needs more than the %zu bytes of scratch",
                    (size_t)KM_SCRATCH_BYTES);
    hipLaunchKernelGGL(k_na_clear, dim3(1), dim3(256), 0, s, (uint32_t *)ctl, (int)(sizeof(km_control) / 4));
    HIPCHK(c, hipGetLastError());
    if (fam == FAM_MFMA_FUSED) {
        HIPCHK(c, km_launch_mfma(mp, 1, X, rows, d, C, k, labels, best, psum, pcomp, 0, ctl, nullptr, nullptr,
                                 KM_LSTATE_NONE, nullptr, s));
    } else if (fam == FAM_LOWD) {
        HIPCHK(c, km_launch_lowd(lp, X, rows, d, C, k, labels, best, psum, pcomp, 0, nullptr, s));
    } else {
        HIPCHK(c, km_launch_assign_rows(X, rows, d, C, k, labels, best, nullptr, s));
        HIPCHK(c, km_launch_accum_generic(ap, X, rows, d, labels, best, k, psum, pcomp, 0, nullptr, s));
    }
    HIPCHK(c, km_launch_reduce_finish(psum, pcomp, nrb, kw, S, red, k, d, totals, nullptr, ctl, 0, 0.0, 0, nullptr, s));
    if (fam == FAM_MFMA_FUSED) {
        // per-cluster best sums: [count, best] accumulated from this pass's labels and best (as km_pass does)
        const int S2 = km_reduce_splits(p2.nrb, kw2, c->dev.cus);
        float *ps2 = nullptr, *pc2 = nullptr;
        double *red2 = nullptr, *tot2 = nullptr;
        if (!sc.take(&ps2, (size_t)p2.nrb * kw2) || !sc.take(&pc2, (size_t)p2.nrb * kw2) ||
            !sc.take(&red2, (size_t)S2 * kw2) || !sc.take(&tot2, (size_t)kw2))
            return fail(c, KM_EINVAL, "km_pass_noalloc: the pass needs more than the %zu bytes of scratch",
                        (size_t)KM_SCRATCH_BYTES);
        HIPCHK(c, km_launch_accum_generic(p2, nullptr, rows, 0, labels, best, k, ps2, pc2, 0, nullptr, s));
        HIPCHK(c, km_launch_reduce_finish(ps2, pc2, p2.nrb, kw2, S2, red2, k, 0, tot2, nullptr, ctl, 0, 0.0, 0, nullptr, s));
        hipLaunchKernelGGL(k_na_best_col, dim3((unsigned)((k + 255) / 256)), dim3(256), 0, s, tot2, k, d + 2, totals);
        HIPCHK(c, hipGetLastError());
    }
    c->last_path = family_path(fam);
    return KM_OK;
}

// ------------------------------------------------------------------ per-centre bounds

extern "C" int32_t km_bounds(km_ctx *c, double max_visited) {
    if (!c) return KM_EINVAL;
    if (!(max_visited >= 0.0 && max_visited <= 1.0))
        return fail(c, KM_EINVAL, "max_visited must be a fraction in [0, 1], got %g", max_visited);
    c->bnd_max_visited = max_visited;
    return KM_OK;
}

extern "C" int32_t km_bounds_info(km_ctx *c, int64_t *passes_tracked, int64_t *passes_on_bounds, int64_t *builds,
                                  double *last_fraction) {
    if (!c) return KM_EINVAL;
    km_bnd st{};
    if (c->bnd_valid && c->bnd_st.p) {
        HIPCHK(c, hipSetDevice(c->device));
        HIPCHK(c, hipMemcpyAsync(&st, c->bnd_st.p, sizeof st, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
    }
    if (passes_tracked) *passes_tracked = (int64_t)st.n_tracked;
    if (passes_on_bounds) *passes_on_bounds = (int64_t)st.n_bounds;
    if (builds) *builds = (int64_t)st.n_builds;
    if (last_fraction) *last_fraction = c->bnd_valid ? st.last_frac : 1.0;
    return KM_OK;
}

// ------------------------------------------------------------------ timing

extern "C" int32_t km_profile(km_ctx *c, int32_t enable) {
    if (!c) return KM_EINVAL;
    harvest(c);
    for (int i = 0; i < KK_COUNT; i++) {
        c->prof_ms[i] = 0.0;
        c->prof_n[i] = 0;
    }
    c->pass_ms.clear();
    c->prof = enable != 0;
    return KM_OK;
}

extern "C" int32_t km_profile_read(km_ctx *c, int32_t kernel, double *ms_total, int64_t *launches) {
    if (!c) return KM_EINVAL;
    if (kernel < 0 || kernel >= KK_COUNT) return fail(c, KM_EINVAL, "kernel id %d out of range", kernel);
    harvest(c);
    if (ms_total) *ms_total = c->prof_ms[kernel];
    if (launches) *launches = c->prof_n[kernel];
    return KM_OK;
}

extern "C" int64_t km_profile_passes(km_ctx *c, double *ms, int64_t cap) {
    if (!c) return KM_EINVAL;
    const int64_t n = (int64_t)c->pass_ms.size();
    if (ms)
        for (int64_t i = 0; i < std::min(n, cap); i++) ms[i] = c->pass_ms[i];
    return n;
}

extern "C" int32_t km_stream_probe(km_ctx *c, int64_t bytes, int32_t reps, double *gbps) {
    if (!c) return KM_EINVAL;
    if (bytes < ((int64_t)1 << 24) || bytes % 16 != 0)
        return fail(c, KM_EINVAL, "the probe reads a multiple of 16 bytes, at least 16 MiB (got %lld)", (long long)bytes);
    if (reps < 1 || !gbps) return fail(c, KM_EINVAL, "reps must be positive and gbps not null");
    HIPCHK(c, hipSetDevice(c->device));
    const int cfg[] = {2, 4, 8, 16};   // blocks of 256 threads per CU
    const int max_blocks = c->dev.cus * 16;
    void *x = nullptr;
    float *out = nullptr;
    HIPCHK(c, hipMalloc(&x, (size_t)bytes));
    hipError_t e = hipMalloc((void **)&out, (size_t)max_blocks * 256 * sizeof(float));
    hipEvent_t a = nullptr, b = nullptr;
    if (e == hipSuccess) e = hipMemsetAsync(x, 0, (size_t)bytes, c->stream);
    if (e == hipSuccess) e = hipEventCreate(&a);
    if (e == hipSuccess) e = hipEventCreate(&b);
    double best = 0.0;
    std::vector<float> t(reps);
    for (int blocks_per_cu : cfg) {
        const int blocks = c->dev.cus * blocks_per_cu;
        for (int w = 0; w < 3 && e == hipSuccess; w++) e = km_launch_stream_read(x, bytes, out, blocks, c->stream);
        for (int i = 0; i < reps && e == hipSuccess; i++) {
            e = hipEventRecord(a, c->stream);
            if (e == hipSuccess) e = km_launch_stream_read(x, bytes, out, blocks, c->stream);
            if (e == hipSuccess) e = hipEventRecord(b, c->stream);
            if (e == hipSuccess) e = hipEventSynchronize(b);
            if (e == hipSuccess) e = hipEventElapsedTime(&t[i], a, b);
        }
        if (e != hipSuccess) break;
        std::vector<float> s = t;
        std::nth_element(s.begin(), s.begin() + reps / 2, s.end());
        best = std::max(best, (double)bytes / (s[reps / 2] * 1e-3) / 1e9);
    }
    (void)hipStreamSynchronize(c->stream);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    (void)hipFree(out);
    (void)hipFree(x);
    if (e != hipSuccess)
        return fail(c, e == hipErrorOutOfMemory ? KM_ENOMEM : KM_EDEVICE, "stream probe failed: %s", hipGetErrorString(e));
    *gbps = best;
    return KM_OK;
}

extern "C" const char *km_kernel_name(int32_t kernel) {
    return (kernel >= 0 && kernel < KK_COUNT) ? km_kernel_names[kernel] : "";
}
