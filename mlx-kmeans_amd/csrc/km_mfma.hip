// MFMA-screened exact assignment for gfx950, fused with the per-cluster accumulation.
//
// Per 32-row tile a wave computes a'_c = |c|^2 - 2 x.c for every centre on the matrix cores, in bf16
// (v_mfma_f32_32x32x16_bf16: A = bf16(-2c), 32 centres x 16 dims; B = bf16(x), 16 dims x 32 rows; C = |c|^2).
// That value is only a screen. A rigorous bound on its error, plus the error bound of the float32 direct form,
// gives a window: every centre whose exact float32 direct-form distance could be the row's minimum has a'_c
// inside it. A row whose window holds the screen's minimiser alone has that label, the rows loop's; the other rows
// (uncommon) are scored against every centre by the whole wave in the rows loop's order (core.py:263-274), ascending
// centre index with a strict '<', so labels and best are the rows loop's bit for bit. This is the reference's
// tiles + margin design (core.py:333-377, 675-784) rebuilt for CDNA4: bf16 matrix cores instead of fp32 simdgroup
// MMA, the window derived for that arithmetic, and no n x k matrix in memory.
//
// Lane layout (wave64, one 32-row tile): lane l holds row n = l & 31 of the tile and half h = l >> 5 of its
// dims: [h*DH, h*DH + DH), DH = DP/2. MFMA K-step s (16 contraction slots) takes dims h*DH + 8s + q (q < 8) from
// lane half h; the A operand (centres) is laid out with the same map, so the contraction runs over every dim.
// Accumulator element v (0..15) of tile t in lane l is centre 32t + 8(v/4) + 4h + (v%4) against row n.
//
// Accumulation (ACCUM), also on the matrix cores: per 64-row block, sums (centres x dims) += onehot^T (centres x
// rows) x rows. The one-hot operand is exact in bf16 (0 or 1, or 0 or 2 where it is read as bytes from LDS, the
// sums then halved exactly at the fold); each row value is split exactly into three bf16
// pieces (split3), so the float32 MFMA accumulators add the float32 row values themselves, rounded only by the
// accumulation. Counts are LDS integer adds (exact, order-free). The block's inertia partial is a per-lane Kahan sum
// of the rows' distances. With BEST every row's distance is the exact direct form (labels, best outputs); without
// it only rows whose window holds several centres get the direct form (from the wave's scan), and the others - whose label
// is the screen's minimiser, exactly the rows loop's label - add their distance in FMA form, which agrees with the
// direct form to float32 rounding. At the end of its rows each wave leaves its accumulators in LDS and the block folds them
// in wave order (Neumaier across waves) into one partial per block; the partials are reduced in a fixed order
// in float64 by a separate kernel. Every step has a fixed order, so the result is the same on every run.
#pragma clang fp contract(off)
#include "km_internal.h"
#include <math.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ the fused kernel
//
// Exactness of the screen. For a row x and centre c let A_c = |c|^2 - 2 x.c (exact reals) and D_c = |x - c|^2 =
// |x|^2 + A_c. The matrix cores give a'_c = sum_j bf16(x_j) h_j + q_h + q_l, where h_j = bf16(-2 c_j) and
// q_h + q_l is |c|^2 split into two bf16 pieces (q_h = bf16(|c|^2), q_l = bf16(|c|^2 - q_h): relative residual
// 2^-16). bf16 rounding to nearest has unit roundoff u = 2^-8 (1 + 2^-8 rounds to 1), so bf16(x_j) = x_j (1 + d) and
// h_j = -2 c_j (1 + e) with |d|, |e| <= 2^-8: each product is -2 x_j c_j (1 + d + e + d e), within
// 2 |x_j| |c_j| (2^-8 + 2^-8 + 2^-16) of the exact one, and sum_j |x_j| |c_j| <= |x| |c|. Products of bf16 values
// are exact in float32 and the float32 accumulation of NACC = DP + 2 terms adds at most gamma_NACC times their
// absolute sum. With bf16 denormal flushing covered by FLUSH,
//     |a'_c - A_c| <= E = BETA |x| max|c| + GAM2 max|c|^2 + FLUSH (|x| + max|c|) + TINY      (uniform in c),
//     BETA = 2 (2^-8 + 2^-8 + 2^-16) + 2.04 gamma_NACC,   GAM2 = 1.01 gamma_NACC + 2^-16 + 2^-23.
// (A second bf16 piece of -2c, the residual, would shrink BETA's second 2^-8 to 2^-16 for one more MFMA per
// K-step; the window it narrows is already wide of almost every row's runner-up, and the MFMAs are not free.)
// The float32 direct form s_c of the rows loop satisfies |s_c - D_c| <= g D_c + eta, g = gamma_{D+2}. A centre c
// can hold the row's minimum only if s_c <= s_m for the screen's minimiser m, which forces
//     a'_c - a'_m <= 2E + 2 g/(1-g) D_m + tiny,   D_m <= |x|^2 + a'_m + E,
// so every centre outside T = a'_m + that margin is ruled out, and rescoring the ones inside in ascending index
// with a strict '<' returns exactly the rows loop's label and best. The screen keys carry a local index in
// their low IB mantissa bits (a relative perturbation of at most RHO), which the test absorbs.

__device__ __forceinline__ uint32_t u32(float v) { return __float_as_uint(v); }

// v_min_f32 as written: fminf would first canonicalise each input (one more instruction per screen value). A key
// that is NaN (non-finite data) makes the row's minimum NaN, and such a row takes the full scan.
__device__ __forceinline__ float vmin(float a, float b) {
    float r;
    asm("v_min_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
// v_min3_f32, defined as two v_min_f32 in a row (the same result for every input, NaN included)
__device__ __forceinline__ float vmin3(float a, float b, float c) {
    float r;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float f32(uint32_t v) { return __uint_as_float(v); }

// v_permlane32_swap: lane l < 32 gets (va of lane l, va of lane l+32); lane l >= 32 gets (vb of lane l-32,
// vb of lane l). With va the tile-A value and vb the tile-B value of this lane's half row, every lane receives
// (half 0, half 1) of the row it owns: tile A row l for l < 32, tile B row l-32 for l >= 32.
__device__ __forceinline__ void own_halves(float va, float vb, float &h0, float &h1) {
    const auto r = __builtin_amdgcn_permlane32_swap(u32(va), u32(vb), false, false);
    h0 = f32(r[0]);
    h1 = f32(r[1]);
}
// orders this wave's LDS accesses (every lane's earlier reads and writes before any later one)
__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Error-window constants. u = 2^-24 (float32 unit roundoff); gamma_m = m u / (1 - m u).
__host__ __device__ constexpr double km_gamma(int m) { return m * 5.9604644775390625e-08 / (1.0 - m * 5.9604644775390625e-08); }

template <int D, int KP>
struct Geo {
    static constexpr int DP = (D + 15) / 16 * 16;   // padded dims
    static constexpr int DH = DP / 2;               // dims per lane half
    static constexpr int DS = DP / 16;              // MFMA K-steps over the dims
    static constexpr int AK = DS + 1;               // A-operand K-steps: bf16(-2c), then |c|^2
    static constexpr int KT = KP / 32;              // centre tiles
    static constexpr int IB = KT <= 1 ? 4 : KT <= 2 ? 5 : 6;   // index bits packed into keys (16 KT values)
    static constexpr int CS = DP + 1;               // LDS row stride of the float32 centres, zero past D (odd:
                                                    // lanes reading different centres' rows hit different banks)
    static constexpr int AS = D + 1;                // LDS row stride of the accumulators
};

// This lane's half row as the screen's B operand (bf16, rounded to nearest), and |bf16(x)|^2 of the half row
// from v_dot2_f32_bf16 on the same pairs.
template <int D, int KP>
__device__ __forceinline__ float make_b(const float (&x)[Geo<D, KP>::DH], bf16x8 (&B)[Geo<D, KP>::DS]) {
    using G = Geo<D, KP>;
    float s = 0.0f;
#pragma unroll
    for (int st = 0; st < G::DS; st++) {
#pragma unroll
        for (int q = 0; q < 8; q++) B[st][q] = (__bf16)x[8 * st + q];
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const bf16x2 v = {B[st][2 * p], B[st][2 * p + 1]};
            s = __builtin_amdgcn_fdot2_f32_bf16(v, v, s, false);
        }
    }
    return s;
}

// Screen one 32-row tile: B is this lane's half row. Returns the KT accumulators (16 screen values each).
template <int D, int KP>
__device__ __forceinline__ void screen_tile(const bf16x8 (&B)[Geo<D, KP>::DS], const bf16x8 (&Aop)[Geo<D, KP>::KT][Geo<D, KP>::AK],
                                            const bf16x8 &Bone, f32x16 (&a)[Geo<D, KP>::KT]) {
    using G = Geo<D, KP>;
    const f32x16 zero = {};
#pragma unroll
    for (int t = 0; t < G::KT; t++) {
        a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Aop[t][0], B[0], zero, 0, 0, 0);
#pragma unroll
        for (int s = 1; s < G::DS; s++) a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Aop[t][s], B[s], a[t], 0, 0, 0);
        a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Aop[t][G::DS], Bone, a[t], 0, 0, 0);
    }
}

// screen_tile with the centre operand's dims K-steps from LDS (Alds[(t DS + s) 64 + lane], shared by the
// workgroup's waves) and its |c|^2 K-step (Acsq) in registers
template <int D, int KP>
__device__ __forceinline__ void screen_tile_lds(const bf16x8 (&B)[Geo<D, KP>::DS], const bf16x8 *Alds, int lane,
                                                const bf16x8 (&Acsq)[Geo<D, KP>::KT], const bf16x8 &Bone,
                                                f32x16 (&a)[Geo<D, KP>::KT]) {
    using G = Geo<D, KP>;
    const f32x16 zero = {};
#pragma unroll
    for (int t = 0; t < G::KT; t++) {
        a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Alds[(t * G::DS) * 64 + lane], B[0], zero, 0, 0, 0);
#pragma unroll
        for (int s = 1; s < G::DS; s++)
            a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Alds[(t * G::DS + s) * 64 + lane], B[s], a[t], 0, 0, 0);
        a[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(Acsq[t], Bone, a[t], 0, 0, 0);
    }
}

template <int D, int KP>
__device__ __forceinline__ void min2_keys(const f32x16 (&a)[Geo<D, KP>::KT], float &m1, float &m2) {
    using G = Geo<D, KP>;
    constexpr uint32_t IMASK = (1u << G::IB) - 1u;
    m1 = 3.4e38f;
    m2 = 3.4e38f;
    // two keys at a time: the smallest of {m1, m2, a, b} is min3(m1, a, b) (m1 <= m2), the second the smaller of
    // m2 and the middle of (m1, a, b): three instructions per pair instead of four
#pragma unroll
    for (int t = 0; t < G::KT; t++)
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
            const float ka = f32((u32(a[t][v]) & ~IMASK) | (uint32_t)(t * 16 + v));
            const float kb = f32((u32(a[t][v + 1]) & ~IMASK) | (uint32_t)(t * 16 + v + 1));
            m2 = vmin(m2, __builtin_amdgcn_fmed3f(m1, ka, kb));
            m1 = vmin3(m1, ka, kb);
        }
}

// Candidate bits of this lane's screen values for one tile: bit (8(v/4) + 4h + v%4) of word t is set when
// a[t][v] <= T2 (the lane's 16 values of centre tile t, for the row its column holds). The values are compared
// unpacked; T2 = T + 4 RHO |T| + tiny covers the packing perturbation, so the set holds every centre the packed-key
// window admits. Compiled code, not inline assembly: the values are matrix-core results, and only the compiler's
// hazard tracking inserts the wait states a vector instruction needs before it may read them.
template <int D, int KP>
__device__ __forceinline__ void cand_bits(const f32x16 (&a)[Geo<D, KP>::KT], float T2, int h,
                                          uint32_t (&w)[Geo<D, KP>::KT]) {
    using G = Geo<D, KP>;
#pragma unroll
    for (int t = 0; t < G::KT; t++) {
        uint32_t m = 0;
#pragma unroll
        for (int v = 15; v >= 0; v--) m = 2u * m + (a[t][v] <= T2 ? 1u : 0u);
        // byte j of the result = nibble j of the 16-bit mask, then shifted into this half's positions
        const uint32_t pq = __builtin_amdgcn_perm(m, m, 0x01010000u);   // bytes b0, b0, b1, b1
        const uint32_t q = ((pq & 0x000f000fu) | ((pq >> 4) & 0x0f000f00u));
        w[t] = q << (4 * h);
    }
}

__device__ __forceinline__ bf16x2 as_bf2(uint32_t v) { return *reinterpret_cast<bf16x2 *>(&v); }
__device__ __forceinline__ uint32_t bf2_u32(bf16x2 v) { return *reinterpret_cast<uint32_t *>(&v); }

// Split x into three bf16 pieces with x = hi + mid + lo exactly, and pack pairs. hi is x truncated to its top 8
// significant bits (never rounds up, so never overflows); r = x - hi is exact in float32 and has at most 16
// significant bits; mid = bf16(r) rounded to nearest; lo = r - mid has at most 8 significant bits, so bf16(lo) is
// exact. The residuals come from v_dot2_f32_bf16 with the pair (-1, 0) or (0, -1): x + (-1) hi + 0, whose products
// are exact and whose sum is representable, so the instruction returns it exactly.
// The two pairs are moved into scalar registers as 32-bit literals: an inline constant in a bf16-pair operand is
// not reliably the pair one means.
__device__ __forceinline__ void split3(const float (&x)[8], bf16x8 &ph, bf16x8 &pm, bf16x8 &pl) {
    uint32_t cl, ch;
    asm("s_mov_b32 %0, 0x0000bf80" : "=s"(cl));
    asm("s_mov_b32 %0, 0xbf800000" : "=s"(ch));
    const bf16x2 nlo = as_bf2(cl), nhi = as_bf2(ch);
    uint32_t h[4], m[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        const float a = x[2 * p], b = x[2 * p + 1];
        h[p] = __builtin_amdgcn_perm(u32(b), u32(a), 0x07060302u);
        const float ra = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(h[p]), nlo, a, false);
        const float rb = __builtin_amdgcn_fdot2_f32_bf16(as_bf2(h[p]), nhi, b, false);
        const bf16x2 mp = {(__bf16)ra, (__bf16)rb};
        m[p] = bf2_u32(mp);
        const float sa = __builtin_amdgcn_fdot2_f32_bf16(mp, nlo, ra, false);
        const float sb = __builtin_amdgcn_fdot2_f32_bf16(mp, nhi, rb, false);
        const bf16x2 lp = {(__bf16)sa, (__bf16)sb};
        l[p] = bf2_u32(lp);
    }
    ph = *reinterpret_cast<bf16x8 *>(h);
    pm = *reinterpret_cast<bf16x8 *>(m);
    pl = *reinterpret_cast<bf16x8 *>(l);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Open rows (several centres in the window) of a 64-row block up to which the whole wave scores each such row
// against every centre (one row at a time, lanes over centres); above it each lane rescores its own row against
// the centres its window lists. The scan costs about 3 D k / 64 + 30 instructions per open row, the lists a
// second screen, the row exchange and 3 D per listed centre: about four open rows apart.
static constexpr int KM_SCAN_ROWS = 4;

// Rows reach LDS by direct global->LDS loads (global_load_lds_dwordx4, non-temporal: a pass reads each row once),
// double-buffered one 64-row block ahead. A block is its 64 rows in order (D floats = NC 16-byte chunks each); one
// load instruction moves 1 KB, i.e. 64/NC whole rows read contiguously, lane i taking the 16 bytes that land at LDS
// offset 16 i. Within each row the chunks are permuted (chunk c of block row r sits at position c ^ swz(r)) so
// that the screen's half-row reads (eight lanes on eight consecutive rows, one chunk each) and the accumulation's
// transposed reads (one dim per lane, one row per read) touch distinct LDS banks (32 banks of 4 bytes). swz
// depends only on the row's low bits, which are compile-time in the transposed reads, so their addresses stay a
// few registers plus immediates.
template <int D>
struct Lay {
    static constexpr int NC = D / 4;           // 16-byte chunks per row
    static constexpr int QI = NC / 2;          // chunks per half row (the screen's reads per tile)
    static constexpr int BUF = 64 * D * 4;     // bytes per 64-row block (NC instructions)
    static constexpr bool SWZ = D == 16 || D == 32 || D == 64;   // rows permuted (NC a power of two)
};

// 48-dim rows (12 chunks) stay in order: a permutation within 12 chunks cannot keep both read patterns on
// distinct banks, and the half-row reads' conflicts (rows 192 bytes apart) cost less than the loads they overlap.
template <int D>
__device__ __forceinline__ int swz(int r) {
    return !Lay<D>::SWZ ? 0 : D == 16 ? ((r >> 1) & 3) : (r & 7);
}

// wait until at most N vector memory operations of this wave are outstanding
template <int N>
__device__ __forceinline__ void vm_wait() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// issue the loads of the 64-row block starting at r0 (rows past r_end read row r_end - 1; never used)
template <int D>
__device__ __forceinline__ void issue_block(const float *__restrict__ X, int64_t r0, int64_t r_end, int lane,
                                            char *buf) {
    using L = Lay<D>;
#pragma unroll
    for (int q = 0; q < L::NC; q++) {
        const int g = q * 64 + lane;           // the 16-byte slot this lane fills
        const int r = g / L::NC, p = g % L::NC;   // block row, position within the row
        int64_t row = r0 + r;
        row = row < r_end ? row : r_end - 1;
        const float *src = X + row * D + 4 * (p ^ swz<D>(r));
        lds_dma16<true>(src, (lds_vptr)(buf + q * 1024));
    }
}

// The same for a block wholly inside the rows: the block's first row as a scalar base, this lane's byte offset
// into instruction q's kilobyte (voff0 for even q, voff1 for odd: they differ only at D = 64) and immediates, so
// issuing takes no vector instructions. The instruction's immediate offset moves the LDS address as well as the
// global one, so M0 carries only the part of q * 1024 the immediate does not.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // M0 in the clobbers: see lds_dma16
template <int D, int Q>
__device__ __forceinline__ void issue_block_inner(const char *blk, uint32_t voff0, uint32_t voff1, uint32_t mb) {
    if constexpr (Q < Lay<D>::NC) {
        const char *sb = blk + (Q / 4) * 4096;   // the immediate offset reaches 4095
        asm volatile("s_add_u32 m0, %1, %4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %2 offset:%3 nt"
                     ::"v"((Q & 1) ? voff1 : voff0), "s"(mb), "s"(sb), "n"((Q % 4) * 1024), "n"((Q / 4) * 4096)
                     : "memory", "m0", "scc");
        issue_block_inner<D, Q + 1>(blk, voff0, voff1, mb);
    }
}
#pragma clang diagnostic pop
template <int D>
__device__ __forceinline__ void issue_block_inner_all(const float *blk, uint32_t voff0, uint32_t voff1, char *buf) {
    const uint32_t mb = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_vptr)buf);
    issue_block_inner<D, 0>(reinterpret_cast<const char *>(blk), voff0, voff1, mb);
}
// this lane's byte offset into the kilobyte of load instruction q (see issue_block)
template <int D>
__device__ __forceinline__ uint32_t issue_voff(int lane, int q) {
    using L = Lay<D>;
    if constexpr (!L::SWZ) return (uint32_t)(16 * lane);   // rows in order: the block's bytes, contiguous
    const int g = q * 64 + lane, r = g / L::NC, p = g % L::NC;   // the slot's block row and position
    return (uint32_t)(r * D * 4 + 16 * (p ^ swz<D>(r)) - 1024 * q);   // its source, from the instruction's kilobyte
}

// this lane's half row of tile `tile` (row ln, dims h DP/2 .. of the dims padded to DP, a multiple of 16; the
// dims past D read as zeros) from a loaded block
template <int D>
__device__ __forceinline__ void read_half(const char *buf, int tile, int lane, float (&x)[(D + 15) / 16 * 8]) {
    using L = Lay<D>;
    constexpr int QH = (D + 15) / 16 * 2;   // chunks per padded half row
    const int ln = lane & 31, h = lane >> 5;
    const int r = 32 * tile + ln, sw = swz<D>(r);
    const char *row = buf + r * (D * 4);
#pragma unroll
    for (int q = 0; q < QH; q++) {
        const int c = h * QH + q;
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (D == (D + 15) / 16 * 16 || c < L::NC) v = *reinterpret_cast<const float4 *>(row + (c ^ sw) * 16);
        x[4 * q] = v.x;
        x[4 * q + 1] = v.y;
        x[4 * q + 2] = v.z;
        x[4 * q + 3] = v.w;
    }
}

// x[row][dim] of a loaded block (row < 64, dim < D)
template <int D>
__device__ __forceinline__ float read_elem(const char *buf, int row, int dim) {
    return *reinterpret_cast<const float *>(buf + row * (D * 4) + (((dim >> 2) ^ swz<D>(row)) * 16) + (dim & 3) * 4);
}

// (Above 32 dims a wave holds 20-32 KB of rows in LDS and two accumulator tiles per centre tile, and 128 centres
// take twice the accumulators, so those run one wave per SIMD: the whole register file.)
//
// Label state across the passes of a fit (LM): 0 none; 1 every row's label is recorded in lout (one byte per row)
// and the pass accumulates every row; 2 the pass reads the previous pass's labels (lprev, brought into LDS with
// the block's rows) and accumulates only the rows whose label changed: +x and +1 for the new cluster, -x and -1
// for the old one (a signed one-hot), so the partials are the change of the totals since the previous pass; a
// 64-row block with no changed row skips the accumulation. The inertia is every row's, in every mode.
template <int D, int KP, int WAVES, bool ACCUM, bool BEST, int LM, bool LIST = true>
__global__ __launch_bounds__(64 * WAVES, (D > 32 || KP >= 128) ? 1 : 2) void k_fused_mfma(
    const float *__restrict__ X, int64_t n, const float *__restrict__ C, int k,
    uint32_t *__restrict__ labels, float *__restrict__ best, float *__restrict__ psum, float *__restrict__ pcomp,
    int rb0, km_control *__restrict__ ctl, const uint8_t *__restrict__ lprev, uint8_t *__restrict__ lout,
    const int32_t *__restrict__ stop, uint32_t *__restrict__ pmask) {
    using G = Geo<D, KP>;
    using L = Lay<D>;
    constexpr int DH = G::DH, DS = G::DS, KT = G::KT, CS = G::CS, W = D + 2;
    constexpr int NT = (D + 31) / 32;                 // 32-dim tiles of the accumulation
    constexpr int FOLD = (KP * 32 * NT + 2 * KP) * 4; // bytes of the end-of-block fold per wave
    // per wave: two block buffers, 64 uint16 labels, the clusters' change bits (TMB bytes) and KP uint32 counts
    // during the loop, the fold after it (the change bits and counts stay in place)
    constexpr int LB = L::BUF + 64;                   // a block buffer: the rows, then their 64 previous labels
    constexpr int TMB = 16;                           // KM_PMASK_WORDS words
    constexpr int LOOPB = 2 * LB + 256 + TMB + 4 * KP;   // + 64 uint16 labels (and 64 old labels)
    constexpr int LX = LM == 2 ? 1 : 0;               // loads per block beyond the rows' (the labels)
    // one-hot bytes in the block buffer once its rows are in registers: KP rows of OHS bytes (64 rows + 8 bytes
    // of padding, so the 32 lanes of a half-wave reading 8 bytes each start on distinct even banks)
    constexpr int OHS = 72, OHB_BYTES = KP * OHS;
    constexpr bool OHB = NT == 1 && OHB_BYTES <= L::BUF;
    constexpr int WBYTES = (LOOPB > FOLD + TMB + 4 * KP) ? LOOPB : FOLD + TMB + 4 * KP;
    constexpr int ABYTES = KT * DS * 64 * 16;         // the screen's centre operand, dims K-steps (per workgroup)
    // each float32 accumulator run covers at most FOLDB blocks (64 FOLDB rows) before it is added into sfold
    constexpr int FOLDB = 16;
    // window constants
    constexpr int NACC = G::DP + 2;
    constexpr float BETA = (float)((2.0 * (0x1p-8 + 0x1p-8 + 0x1p-16) + 2.04 * km_gamma(NACC)) * (1.0 + 0x1p-20));
    constexpr float GAM2 = (float)((1.01 * km_gamma(NACC) + 0x1p-16 + 0x1p-23) * (1.0 + 0x1p-20));
    constexpr float GDIR = (float)(km_gamma(D + 2) / (1.0 - km_gamma(D + 2)) * (1.0 + 0x1p-20));
    constexpr float RHO = (float)(1.01 * (double)(1 << G::IB) * 0x1p-23);
    constexpr float FLUSH = (float)(0x1p-123 * 16.0);
    constexpr float TINY = (float)((G::DP + 2) * 0x1p-118);
    // |x|^2 <= |bf16(x)|^2 / (1 - 2^-8)^2 (each bf16(x_j) is within 2^-8 |x_j|), with slack for the float32
    // accumulation of the v_dot2 sums; XSQ_FLOOR covers products below the smallest normal if they are flushed
    constexpr float XSQ_UP = 1.0079f;
    constexpr float XSQ_FLOOR = (float)(G::DP * 0x1p-126);
    constexpr uint32_t IMASK = (1u << G::IB) - 1u;
    static_assert(D % 8 == 0 && D <= 64 && KP <= 128, "fused kernel serves dims 16-64 (multiples of 8), k <= 128");

    if (stop && *stop) return;

    extern __shared__ float lds[];
    float *Cl = lds;                                  // KP x CS float32 centres
    bf16x8 *Alds = reinterpret_cast<bf16x8 *>(lds + KP * CS);   // KT x DS x 64 lanes of bf16(-2c)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    char *wbase = reinterpret_cast<char *>(lds + KP * CS) + ABYTES + wave * WBYTES;
    uint16_t *L16 = reinterpret_cast<uint16_t *>(wbase + 2 * LB);       // labels of the block (0x4000: no row)
    uint32_t *CNT = reinterpret_cast<uint32_t *>(wbase + WBYTES - 4 * KP);   // rows per centre (this wave)
    uint32_t *TM = CNT - TMB / 4;   // LM 2: bit c set where a changed row of this wave left or joined cluster c
    static_assert(TMB / 4 == KM_PMASK_WORDS && KP <= 32 * KM_PMASK_WORDS, "one bit per cluster");

    // blocks of 64 WAVES rows go round-robin to the workgroups (at any time the whole grid streams one window of
    // the rows), 64 rows per wave
    const int64_t r_end = n, step = (int64_t)gridDim.x * 64 * WAVES;
    int64_t r0 = (int64_t)blockIdx.x * 64 * WAVES + (int64_t)wave * 64;
    const uint32_t voff0 = issue_voff<D>(lane, 0), voff1 = issue_voff<D>(lane, 1);
    if (r0 + 64 <= r_end) issue_block_inner_all<D>(X + r0 * D, voff0, voff1, wbase);
    else if (r0 < r_end) issue_block<D>(X, r0, r_end, lane, wbase);
    if (LM == 2 && r0 < r_end && lane < 4) lds_dma16<true>(lprev + r0 + 16 * lane, (lds_vptr)(wbase + L::BUF));

    for (int e = threadIdx.x; e < KP * CS; e += 64 * WAVES) {
        const int c = e / CS, j = e % CS;
        Cl[e] = (c < k && j < D) ? C[(size_t)c * D + j] : 0.0f;
    }
    const int h = lane >> 5, ln = lane & 31;
    __syncthreads();
    // The screen's A operand from the float32 centres: for centre tile t and K-step s < DS, lane (h, ln) holds
    // bf16(-2 c[32t + ln][h*DH + 8s + q]); K-step DS carries |c|^2 (float32 of the float64 sum over dims
    // ascending; 3e38 for padding centres, never a
    // candidate and finite so packed keys stay ordered) as two bf16 pieces against a B operand of ones, so
    // |c|^2 - 2 x.c comes out of the matrix cores directly. The window needs max |c| (rounded up) and max |c|^2
    // over the real centres.
    bf16x8 Acsq[KT];
    float cn_l = 0.0f, cs_l = 0.0f;
#pragma unroll
    for (int t = 0; t < KT; t++) {
        const int cA = 32 * t + ln;
        const bool real = cA < k;
        double sq = 0.0;
        if (real)
            for (int j = 0; j < D; j++) {
                const double v = Cl[cA * CS + j];
                sq += v * v;
            }
        const float sf = real ? (float)sq : 3.0e38f;
        if (real) {
            cn_l = fmaxf(cn_l, (float)(sqrt(sq) * (1.0 + 1e-6)));
            cs_l = fmaxf(cs_l, sf);
        }
        if (wave == 0) {
#pragma unroll
            for (int st = 0; st < DS; st++) {
                bf16x8 av;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const int j = h * DH + 8 * st + q;
                    const float v = (real && j < D) ? -2.0f * Cl[cA * CS + j] : 0.0f;
                    av[q] = (__bf16)v;
                }
                Alds[(t * DS + st) * 64 + lane] = av;
            }
        }
        const float hi = (float)(__bf16)sf;
#pragma unroll
        for (int q = 0; q < 8; q++) Acsq[t][q] = (__bf16)((h == 0 && q < 2) ? (q == 0 ? hi : sf - hi) : 0.0f);
    }
    for (int off = 32; off > 0; off >>= 1) {
        cn_l = fmaxf(cn_l, __shfl_xor(cn_l, off));
        cs_l = fmaxf(cs_l, __shfl_xor(cs_l, off));
    }
    const float cnmax = cn_l, csqmax = cs_l;
    bf16x8 Bone;
#pragma unroll
    for (int q = 0; q < 8; q++) Bone[q] = (__bf16)((h == 0 && q < 2) ? 1.0f : 0.0f);

    __syncthreads();   // Alds written by wave 0
    float ine_s = 0.0f, ine_c = 0.0f;   // Kahan inertia of this lane's rows
    uint32_t fallback = 0;
    f32x16 sacc[KT][NT], sfold[KT][NT];
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int u = 0; u < NT; u++) {
            sacc[t][u] = f32x16{};
            sfold[t][u] = f32x16{};
        }
    int nblk = 0;
    for (int c = lane; c < KP; c += 64) CNT[c] = 0u;
    if (LM == 2 && lane < TMB / 4) TM[lane] = 0u;
    const uint32_t ones = 0x00010001u, c3f80 = 0x3f803f80u, cneg = 0xc080c080u;

    // the two block buffers alternate by offset (pointer arithmetic keeps the LDS address space visible)
    int cur = 0;
    for (; r0 < r_end; r0 += step, cur ^= LB) {
        const char *buf = wbase + cur;
        // ---- prefetch the next block into the other buffer, then wait for this one
        const int64_t r1 = r0 + step;
        if (r1 < r_end) {
            if (r1 + 64 <= r_end) issue_block_inner_all<D>(X + r1 * D, voff0, voff1, wbase + (cur ^ LB));
            else issue_block<D>(X, r1, r_end, lane, wbase + (cur ^ LB));
            if (LM == 2 && lane < 4) lds_dma16<true>(lprev + r1 + 16 * lane, (lds_vptr)(wbase + (cur ^ LB) + L::BUF));
            vm_wait<L::NC + LX>();
        } else {
            vm_wait<0>();
        }
        const int64_t row = r0 + lane;     // the row this lane owns after the exchange
        const bool valid = row < r_end;
        float xa[DH], xb[DH];
        read_half<D>(buf, 0, lane, xa);
        read_half<D>(buf, 1, lane, xb);
        // ---- screens of tiles A and B
        float m1a, m2a, m1b, m2b, sa, sb;
        {
            bf16x8 B[DS];
            sa = make_b<D, KP>(xa, B);
            f32x16 a[KT];
            screen_tile_lds<D, KP>(B, Alds, lane, Acsq, Bone, a);
            min2_keys<D, KP>(a, m1a, m2a);
        }
        {
            bf16x8 B[DS];
            sb = make_b<D, KP>(xb, B);
            f32x16 a[KT];
            screen_tile_lds<D, KP>(B, Alds, lane, Acsq, Bone, a);
            min2_keys<D, KP>(a, m1b, m2b);
        }
        // ---- the owned row's two halves
        float p0, p1, q0, q1, s0, s1;
        own_halves(m1a, m1b, p0, p1);
        own_halves(m2a, m2b, q0, q1);
        own_halves(sa, sb, s0, s1);
        const float km = fminf(p0, p1);
        const int kh = (p0 <= p1) ? 0 : 1;
        const float k2 = fminf(fmaxf(p0, p1), fminf(q0, q1));
        const uint32_t kmb = u32(km) & IMASK;
        const int kt = (int)kmb >> 4, kv = (int)kmb & 15;
        const int cm = 32 * kt + 8 * (kv >> 2) + 4 * kh + (kv & 3);
        const float xsq_up = __builtin_fmaf(s0 + s1, XSQ_UP, XSQ_FLOOR);
        const float nx = __builtin_sqrtf(xsq_up) * (1.0f + 0x1p-22f);
        const float E = BETA * nx * cnmax + GAM2 * csqmax + FLUSH * (nx + cnmax) + TINY;
        const float akm = km + RHO * fabsf(km);
        const float dm_up = fmaxf(0.0f, xsq_up + akm + E) * (1.0f + 0x1p-20f);
        float T = akm + ((2.0f * E + 2.0f * GDIR * dm_up) * (1.0f + 0x1p-20f) + TINY);
        T = T + 0x1p-22f * fabsf(T);
        const bool unique = (k2 - RHO * fabsf(k2)) > T && cm < k;
        float bst = 0.0f;
        uint32_t bl = unique ? (uint32_t)cm : 0u;
        if (BEST) {
            // ---- every row's exact distance to its label: the lane takes its whole row (rows the window leaves
            // open get theirs from the scan below)
            asm volatile("" ::: "memory");
            float lo[DH], hi[DH];
#pragma unroll
            for (int q = 0; q < DH; q++) own_halves(xa[q], xb[q], lo[q], hi[q]);
            const float *cc = Cl + (unique ? cm : 0) * CS;
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < DH; q++) { const float t = lo[q] - cc[q]; s = s + t * t; }
#pragma unroll
            for (int q = 0; q < DH; q++) { const float t = hi[q] - cc[DH + q]; s = s + t * t; }
            bst = s;
            // the rows loop keeps best = INFINITY and label 0 when no distance compares below it (NaN)
            if (!(s < INFINITY)) { bst = INFINITY; bl = 0; }
        }
        // ---- rows the window leaves open (uncommon: about 0.5 % of rows on 10M x 32, k = 64 blobs with outliers,
        // non-finite rows always): the whole wave scores every centre of each such row in the rows loop's order
        // (dims ascending, lane c taking centres c, c + 64, ... ascending with a strict '<'), then keeps the
        // smallest distance and the lowest index among equal ones - the rows loop's label and best, label 0 and
        // best +inf included when no distance compares below +inf. The row is read from the block buffer by
        // every lane at one address (a broadcast).
        uint64_t need = __ballot(!unique && valid);
        if (LIST && need && __popcll(need) > KM_SCAN_ROWS) {
            // ---- many open rows (data whose distances crowd inside the window): each lane rescores its own row
            // against the centres inside that row's window only. The screen runs again to list them (its values
            // were not kept), each lane takes its whole row, and the direct form runs over the listed centres in
            // ascending order with a strict '<' - the rows loop restricted to every centre that can win.
            asm volatile("" ::: "memory");
            fallback += (!unique && valid) ? 1u : 0u;
            const float T2 = T + (4.0f * RHO * fabsf(T) + TINY);
            const auto tx = __builtin_amdgcn_permlane32_swap(u32(T2), u32(T2), false, false);
            const float Tp = f32(lane < 32 ? tx[1] : tx[0]);   // the partner lane's threshold
            const float TA = lane < 32 ? T2 : Tp, TB = lane < 32 ? Tp : T2;   // tile A's row ln, tile B's row ln
            uint32_t wa[KT], wb[KT], mw[KT];
            {
                bf16x8 B[DS];
                (void)make_b<D, KP>(xa, B);
                f32x16 a[KT];
                screen_tile_lds<D, KP>(B, Alds, lane, Acsq, Bone, a);
                cand_bits<D, KP>(a, TA, h, wa);
            }
            {
                bf16x8 B[DS];
                (void)make_b<D, KP>(xb, B);
                f32x16 a[KT];
                screen_tile_lds<D, KP>(B, Alds, lane, Acsq, Bone, a);
                cand_bits<D, KP>(a, TB, h, wb);
            }
            uint32_t any = 0;
#pragma unroll
            for (int t = 0; t < KT; t++) {
                const auto u = __builtin_amdgcn_permlane32_swap(wa[t], wb[t], false, false);
                uint32_t m = u[0] | u[1];
                const int lim = k - 32 * t;
                if (lim < 32) m &= lim <= 0 ? 0u : ((1u << lim) - 1u);
                mw[t] = (!unique && valid) ? m : 0u;
                any |= m;
            }
            if (!unique && valid && any == 0) {   // nothing finite in the window (non-finite data): every centre
#pragma unroll
                for (int t = 0; t < KT; t++) {
                    const int lim = k - 32 * t;
                    mw[t] = lim >= 32 ? 0xffffffffu : (lim <= 0 ? 0u : ((1u << lim) - 1u));
                }
            }
            float lo[DH], hi[DH];
#pragma unroll
            for (int q = 0; q < DH; q++) own_halves(xa[q], xb[q], lo[q], hi[q]);
            if (!unique && valid) {
                float bv = INFINITY;
                uint32_t bi = 0;
#pragma unroll
                for (int t = 0; t < KT; t++) {
                    uint32_t wv = mw[t];
                    while (wv) {
                        const int c = 32 * t + __builtin_ctz(wv);
                        wv &= wv - 1u;
                        const float *cc = Cl + c * CS;
                        float sc = 0.0f;
#pragma unroll
                        for (int q = 0; q < DH; q++) { const float tq = lo[q] - cc[q]; sc = sc + tq * tq; }
#pragma unroll
                        for (int q = 0; q < DH; q++) { const float tq = hi[q] - cc[DH + q]; sc = sc + tq * tq; }
                        if (sc < bv) {
                            bv = sc;
                            bi = (uint32_t)c;
                        }
                    }
                }
                bst = bv;
                bl = bi;
            }
        } else if (need) {
            asm volatile("" ::: "memory");
            fallback += (!unique && valid) ? 1u : 0u;
            do {
                const int L = __builtin_ctzll(need);
                need &= need - 1;
                const char *rowp = buf + L * (D * 4);
                const int swl = swz<D>(L);
                float bv = INFINITY;
                uint32_t bi = 0;
                for (int c = lane; c < k; c += 64) {
                    const float *cc = Cl + c * CS;
                    float sc = 0.0f;
#pragma unroll
                    for (int p = 0; p < D / 4; p++) {
                        const float4 xq = *reinterpret_cast<const float4 *>(rowp + ((p ^ swl) << 4));
                        const float t0 = xq.x - cc[4 * p], t1 = xq.y - cc[4 * p + 1];
                        const float t2 = xq.z - cc[4 * p + 2], t3 = xq.w - cc[4 * p + 3];
                        sc = sc + t0 * t0;
                        sc = sc + t1 * t1;
                        sc = sc + t2 * t2;
                        sc = sc + t3 * t3;
                    }
                    if (sc < bv) {
                        bv = sc;
                        bi = (uint32_t)c;
                    }
                }
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) {
                    const float ov = __shfl_xor(bv, off);
                    const uint32_t oi = (uint32_t)__shfl_xor((int)bi, off);
                    if (ov < bv || (ov == bv && oi < bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                if (lane == L) {
                    bst = bv;
                    bl = bi;
                }
            } while (need);
        }
        if (!BEST && ACCUM) {
            // inertia of the rows the screen settled alone: |x - c_m|^2 in FMA form on the half-rows each lane
            // holds (the label needs no distance; the sum agrees with the direct form's to float32 rounding)
            const uint32_t cmo = unique ? (uint32_t)cm : 0u;
            const auto sw = __builtin_amdgcn_permlane32_swap(cmo, cmo, false, false);
            const uint32_t cA = lane < 32 ? cmo : sw[0], cB = lane < 32 ? sw[1] : cmo;
            const float *ca = Cl + cA * CS + h * DH, *cbp = Cl + cB * CS + h * DH;
            float pa[4] = {0.0f, 0.0f, 0.0f, 0.0f}, pb[4] = {0.0f, 0.0f, 0.0f, 0.0f};   // four independent chains each
#pragma unroll
            for (int q = 0; q < DH; q++) {
                const float ta = xa[q] - ca[q], tb = xb[q] - cbp[q];
                pa[q & 3] = __builtin_fmaf(ta, ta, pa[q & 3]);
                pb[q & 3] = __builtin_fmaf(tb, tb, pb[q & 3]);
            }
            float s0h, s1h;
            own_halves((pa[0] + pa[1]) + (pa[2] + pa[3]), (pb[0] + pb[1]) + (pb[2] + pb[3]), s0h, s1h);
            if (unique) bst = s0h + s1h;
        }
        // the previous pass's label of the owned row (LM 2), and whether the row changed cluster
        const uint32_t prv = (LM == 2 && valid) ? (uint32_t)reinterpret_cast<const uint8_t *>(buf + L::BUF)[lane] : bl;
        const bool moved = LM == 2 ? (valid && prv != bl) : valid;
        if (valid) {
            if (labels) labels[row] = bl;
            if (BEST && best) best[row] = bst;
            if (LM == 1 || (LM == 2 && moved)) lout[row] = (uint8_t)bl;
        }
        if (ACCUM) {
            // ---- accumulation on the matrix cores: sums (centres x dims) += onehot^T (centres x rows) x rows
            if (valid) {
                const float y = bst - ine_c;
                const float tt = ine_s + y;
                ine_c = (tt - ine_s) - y;
                ine_s = tt;
            }
            if (LM != 2 || __ballot(moved)) {
            if (moved) {
                atomicAdd(&CNT[bl], 1u);   // integer adds: the order does not matter
                if (LM == 2) {
                    atomicAdd(&CNT[prv], 0xffffffffu);   // -1: the row left its old cluster
                    atomicOr(&TM[bl >> 5], 1u << (bl & 31));
                    atomicOr(&TM[prv >> 5], 1u << (prv & 31));
                }
            }
            if constexpr (OHB) {
                // The block's rows in the accumulation's layout (lane = one dim, eight rows per K-step) go to
                // registers first; then the block buffer holds the one-hot bytes: byte [c][r] = 0x40, the high
                // byte of bf16 2.0, where row r has label c (one byte write per row instead of a compare per
                // (row, centre)); the sums come out doubled, exactly, and the fold halves them.
                float xv[4][8];
#pragma unroll
                for (int ks = 0; ks < 4; ks++)
#pragma unroll
                    for (int i = 0; i < 8; i++) xv[ks][i] = (ln < D) ? read_elem<D>(buf, 16 * ks + 8 * h + i, ln) : 0.0f;
                wave_sync();
                char *ohb = wbase + cur;
#pragma unroll
                for (int i = lane; i < OHB_BYTES / 16; i += 64) reinterpret_cast<uint4 *>(ohb)[i] = uint4{0u, 0u, 0u, 0u};
                wave_sync();
                if (moved) {
                    ohb[bl * OHS + lane] = (char)0x40;
                    if (LM == 2) ohb[prv * OHS + lane] = (char)0xc0;   // -2.0: the row leaves its old cluster
                }
                wave_sync();
#pragma unroll
                for (int ks = 0; ks < 4; ks++) {
                    bf16x8 OH[KT];
#pragma unroll
                    for (int t = 0; t < KT; t++) {
                        const uint2 w = *reinterpret_cast<const uint2 *>(ohb + (32 * t + ln) * OHS + 16 * ks + 8 * h);
                        const uint32_t o[4] = {__builtin_amdgcn_perm(w.y, w.x, 0x010c000cu),
                                               __builtin_amdgcn_perm(w.y, w.x, 0x030c020cu),
                                               __builtin_amdgcn_perm(w.y, w.x, 0x050c040cu),
                                               __builtin_amdgcn_perm(w.y, w.x, 0x070c060cu)};
                        OH[t] = *reinterpret_cast<const bf16x8 *>(o);
                    }
                    bf16x8 ph, pm, pl;
                    split3(xv[ks], ph, pm, pl);
#pragma unroll
                    for (int t = 0; t < KT; t++) {
                        sacc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], ph, sacc[t][0], 0, 0, 0);
                        sacc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], pm, sacc[t][0], 0, 0, 0);
                        sacc[t][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], pl, sacc[t][0], 0, 0, 0);
                    }
                }
            } else {
            L16[lane] = moved ? (uint16_t)bl : (uint16_t)0x4000u;
            if (LM == 2) L16[64 + lane] = moved ? (uint16_t)prv : (uint16_t)0x4000u;
            wave_sync();
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const int rbase = 16 * ks + 8 * h;           // this lane's 8 rows of the K-step
                const uint4 lp = *reinterpret_cast<const uint4 *>(L16 + rbase);   // 8 uint16 labels
                const uint32_t lab2[4] = {lp.x, lp.y, lp.z, lp.w};
                uint32_t old2[4] = {0u, 0u, 0u, 0u};
                if (LM == 2) {
                    const uint4 lq = *reinterpret_cast<const uint4 *>(L16 + 64 + rbase);   // their old labels
                    old2[0] = lq.x;
                    old2[1] = lq.y;
                    old2[2] = lq.z;
                    old2[3] = lq.w;
                }
                bf16x8 OH[KT];
#pragma unroll
                for (int t = 0; t < KT; t++) {
                    const uint32_t mm = (uint32_t)(32 * t + ln) * 0x00010001u;
                    uint32_t o[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) {
                        // per 16-bit half: y = min(label ^ m, 1) is 0 exactly on a match; onehot = 0x3f80 - y * 0x3f80
                        uint32_t y, oh;
                        asm("v_pk_min_u16 %0, %1, %2" : "=v"(y) : "v"(lab2[p] ^ mm), "v"(ones));
                        asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(oh) : "v"(y), "v"(cneg), "v"(c3f80));
                        if (LM == 2) {   // -1 (0xbf80) where the row's old label matches; a moved row matches one
                            uint32_t y2, oh2;
                            asm("v_pk_min_u16 %0, %1, %2" : "=v"(y2) : "v"(old2[p] ^ mm), "v"(ones));
                            asm("v_pk_mad_u16 %0, %1, %2, %3" : "=v"(oh2) : "v"(y2), "v"(cneg), "v"(c3f80));
                            oh |= oh2 | ((oh2 & 0x00800080u) << 8);   // 0x3f80 -> 0xbf80 (bit 7 marks a match)
                        }
                        o[p] = oh;
                    }
                    OH[t] = *reinterpret_cast<bf16x8 *>(o);
                }
#pragma unroll
                for (int u = 0; u < NT; u++) {
                    float xv[8];
                    const int col = 32 * u + ln;
#pragma unroll
                    for (int i = 0; i < 8; i++) xv[i] = (col < D) ? read_elem<D>(buf, rbase + i, col) : 0.0f;
                    bf16x8 ph, pm, pl;
                    split3(xv, ph, pm, pl);
#pragma unroll
                    for (int t = 0; t < KT; t++) {
                        sacc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], ph, sacc[t][u], 0, 0, 0);
                        sacc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], pm, sacc[t][u], 0, 0, 0);
                        sacc[t][u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(OH[t], pl, sacc[t][u], 0, 0, 0);
                    }
                }
            }
            }
            }   // a block with no changed row (LM 2) skips the accumulation
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            if (++nblk == FOLDB) {   // bound the float32 run: add it into sfold and start again
                nblk = 0;
#pragma unroll
                for (int t = 0; t < KT; t++)
#pragma unroll
                    for (int u = 0; u < NT; u++) {
                        sfold[t][u] += sacc[t][u];
                        sacc[t][u] = f32x16{};
                    }
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int u = 0; u < NT; u++) sacc[t][u] += sfold[t][u];

    if (fallback) atomicAdd((unsigned long long *)&ctl->fallback_rows, (unsigned long long)fallback);
    if (!ACCUM) return;

    // ---- fold: each wave leaves its sums and counts in its own buffers; the block folds them in wave order
    __shared__ float ine_w[WAVES * 2];
    {
        float s = ine_s, c = -ine_c;   // Kahan: the true sum is s - carry
        for (int off = 32; off > 0; off >>= 1) {
            const float so = __shfl_xor(s, off), co = __shfl_xor(c, off);
            const float a0 = (lane & off) ? so : s, a1 = (lane & off) ? s : so;
            const float c0 = (lane & off) ? co : c, c1 = (lane & off) ? c : co;
            const float tt = a0 + a1;
            const float err = (fabsf(a0) >= fabsf(a1)) ? ((a0 - tt) + a1) : ((a1 - tt) + a0);
            s = tt;
            c = c0 + c1 + err;
        }
        if (lane == 0) {
            ine_w[wave * 2] = s;
            ine_w[wave * 2 + 1] = c;
        }
    }
    float *F = reinterpret_cast<float *>(wbase);                      // KP x (32 NT) sums of this wave
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int t = 0; t < KT; t++)
#pragma unroll
        for (int u = 0; u < NT; u++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const int c = 32 * t + 8 * (v >> 2) + 4 * h + (v & 3);
                F[c * (32 * NT) + 32 * u + ln] = OHB ? 0.5f * sacc[t][u][v] : sacc[t][u][v];
            }
    __syncthreads();
    const int64_t kw = (int64_t)k * W;
    float *ps = psum + (int64_t)(rb0 + blockIdx.x) * kw;
    float *pc = pcomp + (int64_t)(rb0 + blockIdx.x) * kw;
    const char *base = reinterpret_cast<const char *>(lds + KP * CS) + ABYTES;   // the first wave's region
    // LM 2 with pmask: only the rows of clusters a changed row left or joined (and cluster 0's, which carries the
    // inertia) are written, and the block's mask says which; every other row of its partials is zero
    const bool masked = LM == 2 && pmask != nullptr;
    __shared__ uint32_t bmask[TMB / 4];
    if (masked) {
        if (threadIdx.x < TMB / 4) {
            uint32_t m = threadIdx.x == 0 ? 1u : 0u;
            for (int w = 0; w < WAVES; w++)
                m |= reinterpret_cast<const uint32_t *>(base + w * WBYTES + WBYTES - 4 * KP - TMB)[threadIdx.x];
            bmask[threadIdx.x] = m;
            pmask[(int64_t)(rb0 + blockIdx.x) * KM_PMASK_WORDS + threadIdx.x] = m;
        }
        __syncthreads();
    }
    for (int e = threadIdx.x; e < k * W; e += 64 * WAVES) {
        const int c = e / W, col = e % W;
        if (masked && !((bmask[c >> 5] >> (c & 31)) & 1u)) continue;
        float s = 0.0f, cc = 0.0f;
        if (col == 0) {
            uint32_t tot = 0;
            for (int w = 0; w < WAVES; w++)
                tot += reinterpret_cast<const uint32_t *>(base + w * WBYTES + WBYTES - 4 * KP)[c];
            s = (float)(int32_t)tot;   // a change of the count (LM 2) may be negative
        } else if (col == 1) {
            if (c == 0) {
                for (int w = 0; w < WAVES; w++) {
                    const float v = ine_w[2 * w];
                    const float tt = s + v;
                    cc += (fabsf(s) >= fabsf(v)) ? ((s - tt) + v) : ((v - tt) + s);
                    cc += ine_w[2 * w + 1];
                    s = tt;
                }
            }
        } else {
            const int jj = col - 2;
            for (int w = 0; w < WAVES; w++) {
                const float v = reinterpret_cast<const float *>(base + w * WBYTES)[c * (32 * NT) + jj];
                const float tt = s + v;
                cc += (fabsf(s) >= fabsf(v)) ? ((s - tt) + v) : ((v - tt) + s);
                s = tt;
            }
        }
        ps[e] = s;
        pc[e] = cc;
    }
}

// ------------------------------------------------------------------ planning and launch

typedef void (*fused_fn)(const float *, int64_t, const float *, int, uint32_t *, float *, float *, float *,
                         int, km_control *, const uint8_t *, uint8_t *, const int32_t *, uint32_t *);

// One entry per served shape: 4-wave blocks where the device gives a block enough LDS, 2-wave blocks otherwise.
// Per block size: the pass without label state, with the rows' exact distances ("b": labels and best outputs),
// recording the labels ("r"), accumulating only the rows whose label changed ("i"), and the last without the
// candidate lists for crowded waves ("s": the whole-wave scan for every open row; a smaller kernel, for data whose
// open rows are rare).
struct fused_entry {
    int d, kp;
    fused_fn acc4, acc4b, acc4r, acc4i, acc4s, acc2, acc2b, acc2r, acc2i, acc2s;
};

#define KM_FUSED(DD, KK)                                                                                     \
    {DD, KK, k_fused_mfma<DD, KK, 4, true, false, 0>, k_fused_mfma<DD, KK, 4, true, true, 0>,              \
     k_fused_mfma<DD, KK, 4, true, false, 1>, k_fused_mfma<DD, KK, 4, true, false, 2>,                     \
     k_fused_mfma<DD, KK, 4, true, false, 2, false>,                                                       \
     k_fused_mfma<DD, KK, 2, true, false, 0>, k_fused_mfma<DD, KK, 2, true, true, 0>,                      \
     k_fused_mfma<DD, KK, 2, true, false, 1>, k_fused_mfma<DD, KK, 2, true, false, 2>,                     \
     k_fused_mfma<DD, KK, 2, true, false, 2, false>}

static fused_entry g_fused[] = {
    KM_FUSED(16, 32), KM_FUSED(16, 64), KM_FUSED(16, 128),
    KM_FUSED(24, 32), KM_FUSED(24, 64), KM_FUSED(24, 128),
    KM_FUSED(32, 32), KM_FUSED(32, 64), KM_FUSED(32, 128),
    KM_FUSED(40, 32), KM_FUSED(40, 64),
    KM_FUSED(48, 32), KM_FUSED(48, 64),
    KM_FUSED(56, 32), KM_FUSED(56, 64),
    KM_FUSED(64, 32), KM_FUSED(64, 64),
};
#undef KM_FUSED

// mirrors the kernel's layout: centres, the screen operand, then per wave max(two block buffers with their labels
// + label staging + change bits + counts, fold + change bits + counts)
static size_t lds_for(int d, int kp, int waves) {
    const size_t tmb = 4 * KM_PMASK_WORDS;
    const size_t loop = 2 * ((size_t)(64 * d * 4) + 64) + 256 + tmb + 4 * (size_t)kp;
    const size_t fold = ((size_t)kp * 32 * ((d + 31) / 32) + 2 * (size_t)kp) * sizeof(float) + tmb + 4 * (size_t)kp;
    const size_t abytes = (size_t)(kp / 32) * ((d + 15) / 16) * 64 * 16;
    return (size_t)kp * ((d + 15) / 16 * 16 + 1) * sizeof(float) + abytes + waves * (loop > fold ? loop : fold);
}

static const fused_entry *find_fused(int d, int k) {
    const int kp = k <= 32 ? 32 : k <= 64 ? 64 : k <= 128 ? 128 : 0;
    for (auto &e : g_fused)
        if (e.d == d && e.kp == kp) return &e;
    return nullptr;
}

km_mfma_plan km_plan_mfma(const km_device_info &dev, int64_t n, int d, int k, int64_t max_blocks) {
    km_mfma_plan pl{};
    const fused_entry *fe = find_fused(d, k);
    if (!fe || n < 1) return pl;
    int waves = 4;
    size_t lds = lds_for(d, fe->kp, 4);
    if (lds > dev.lds_max) {
        waves = 2;
        lds = lds_for(d, fe->kp, 2);
        if (lds > dev.lds_max) return pl;
    }
    fused_fn fn = waves == 4 ? fe->acc4 : fe->acc2;
    if (lds > 65536) {
        const fused_fn all[5] = {fn, waves == 4 ? fe->acc4b : fe->acc2b, waves == 4 ? fe->acc4r : fe->acc2r,
                                 waves == 4 ? fe->acc4i : fe->acc2i, waves == 4 ? fe->acc4s : fe->acc2s};
        for (fused_fn f : all)
            (void)hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void *)fn, 64 * waves, lds) != hipSuccess || occ < 1)
        occ = 1;
    pl.ok = 1;
    pl.kpad = fe->kp;
    pl.dpad = (d + 15) / 16 * 16;
    pl.lds = lds;
    pl.waves = waves;
    const int64_t slots = (int64_t)dev.cus * occ;
    const int64_t unit = 64 * waves;
    const int64_t units = (n + unit - 1) / unit;
    int64_t nrb = units < slots ? units : slots;
    if (max_blocks > 0 && nrb > max_blocks) nrb = max_blocks;
    if (nrb < 1) nrb = 1;
    pl.nrb = (int)nrb;
    pl.rbs = (units + nrb - 1) / nrb * unit;   // at most this many rows per block
    return pl;
}

hipError_t km_launch_mfma(const km_mfma_plan &pl, int want_best, const float *X, int64_t n, int d, const float *C,
                          int k, uint32_t *labels, float *best, float *psum, float *pcomp, int rb0, km_control *ctl,
                          const uint8_t *lprev, uint8_t *lout, int lmode, const int32_t *stop, hipStream_t s,
                          int scan_only, uint32_t *pmask) {
    const fused_entry *fe = find_fused(d, k);
    if (!fe || !pl.ok) return hipErrorInvalidValue;
    if (lmode != 0 && (want_best || !lout || (lmode == 2 && !lprev))) return hipErrorInvalidValue;
    if (lmode != 2) pmask = nullptr;   // only the change-only passes leave rows of partials unwritten
    const bool w4 = pl.waves == 4;
    fused_fn fn = want_best ? (w4 ? fe->acc4b : fe->acc2b)
                  : lmode == 1 ? (w4 ? fe->acc4r : fe->acc2r)
                  : lmode == 2 ? (scan_only ? (w4 ? fe->acc4s : fe->acc2s) : (w4 ? fe->acc4i : fe->acc2i))
                               : (w4 ? fe->acc4 : fe->acc2);
    hipLaunchKernelGGL(fn, dim3(pl.nrb), dim3(64 * pl.waves), pl.lds, s, X, n, C, k, labels, best, psum,
                       pcomp, rb0, ctl, lprev, lout, stop, pmask);
    return hipGetLastError();
}
