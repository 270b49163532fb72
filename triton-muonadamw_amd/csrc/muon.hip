// Muon step for gfx950: momentum -> Newton-Schulz (bf16 MFMA) -> update.
//
// Launch sequence for one batch of equal-shaped matrices (mamw_muon_step):
//   1. muon_prep_kernel   momentum lerp, Nesterov blend, bf16 cast; writes
//                         X^T (n x m, zero-padded: a tall parameter's rows
//                         are X^T rows, a wide one is transposed through LDS)
//                         and one fp32 sum of squares per prep unit of
//                         32 x 128 parameter elements.
//   2. muon_norm_kernel   fixed-order reduction of those partials ->
//                         inv[b] = 1 / max(bf16(||X||_F), eps).
//   3. muon_scale_kernel  XT = bf16(XT * inv[b]) in place (torch's
//                         X.div_(norm) rounding point).
//   4. ns_steps x { GRAM: A = X X^T,  POLY: B = b A + c A A,  UPDATE: X = a X + B X }
//      with X held as XT only: the Gram reads XT k-major (LDS transpose reads)
//      and UPDATE writes the next XT.  The last iteration's UPDATE is APPLY:
//      its epilogue transposes back and writes param = param*(1-lr*wd) - slr*X.
// All GEMMs are C = A_op * B_op^T over operands stored with the reduction
// index contiguous (A for A A since A is symmetric, B and XT for B X), except
// the Gram, whose operand XT has the reduction index as its row.  Workspace
// matrices too large for 31-bit buffer offsets are row-major instead, and
// there X itself is kept beside XT for a row-major Gram: prep writes X and
// the scale kernel writes both X and XT = bf16(X * inv[b])^T.
#include <mutex>
#include <type_traits>

#include "mamw_device.h"
#include "mamw_launch.h"

namespace mamw {
namespace {

constexpr int kGemmThreads = 256;
constexpr int kBK = 64;

enum GemmMode { MODE_GRAM = 0, MODE_POLY = 1, MODE_UPDATE = 2, MODE_APPLY = 3 };

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t* lds_i16x4_ptr_t;

// gfx950 LDS transpose read (ds_read_b64_tr_b16) of 16-bit elements: within
// each group of 16 lanes, lane j names 4 consecutive elements c_j[0..3];
// lane i receives c_{4r + i/4}[i%4] for r = 0..3.
__device__ __forceinline__ uint2 lds_read_tr16(const uint16_t* p) {
    const i16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_ptr_t)(lds_ptr_t)(p));
    return __builtin_bit_cast(uint2, v);
}

// The same read issued as inline assembly, which the compiler's wait-count
// pass does not see: the builtin's memory operand carries no alias scope, so
// the pass would make every such read inside the GEMM loop wait for all LDS
// DMA in flight (vmcnt(0)).  The caller waits for the result itself
// (s_waitcnt lgkmcnt) before using it.
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// `addr` is an LDS byte address, `off` a byte offset that must be a constant
// once the caller is inlined and unrolled (it becomes the instruction's
// immediate, 0..65535).
__device__ __forceinline__ uint2 lds_read_tr16_untracked(uint32_t addr, int off) {
    u32x2_t v;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(off));
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_ptr_t)(p)));
}

// ---------------------------------------------------------------------------
// Prep: one tile of 64 x 128 parameter elements per block, two prep units
// of 32 rows (parameter rows read in 512-byte runs; 64 x 64 tiles measured 6%
// slower).  The output is X^T (k-blocked workspace) or X (row-major): where
// parameter rows are output rows (X^T of a tall matrix, X of a wide one) the
// tile is written as it stands, otherwise it is transposed through LDS into
// 128 full 128-byte output rows.

struct PrepArgs {
    uint16_t* x;    // [batch][mp][np], k-blocked when xkb (see xoff)
    uint16_t* xt;   // [batch][np][mp], k-blocked when xkb
    float* part;    // [batch][prep_tiles]
    int64_t mp, np;
    int64_t prep_tiles;
    int tiles_j;    // np / 64 (the scale kernel's tiles per 128-row band of X)
    float w_mom;    // 1 - beta   (lerp weight of the momentum update)
    float w_nest;   // beta       (lerp weight of the Nesterov blend)
    int xkb;        // workspace matrices are k-blocked
    int xt_direct;  // prep writes X^T and the scale pass rescales it in place
                    // (else prep writes X and the scale pass writes X and X^T)
    // Gradient-scaler step (NULL otherwise): gradients are divided by
    // *grad_scale; a non-zero *found_inf leaves the momentum (and, in the
    // apply kernels, the parameters) untouched.
    const float* grad_scale;
    const float* found_inf;
};

// Offset of element [r][c] of a rows x cols workspace matrix (X: mp x np,
// X^T: np x mp, A and B: mp x mp).  Row-major, or k-blocked: column panels of
// 64 (one GEMM k step) stacked, each rows x 64 row-major, so one k step of a
// 256-row operand tile is one contiguous 32 KB block and a 256 x 256 output
// tile is four contiguous 32 KB blocks.
__device__ __forceinline__ int64_t xoff(int xkb, int64_t rows, int64_t cols, int64_t r, int64_t c) {
    return xkb ? (((c >> 6) * rows + r) << 6) + (c & 63) : r * cols + c;
}

template <bool NESTEROV>
__global__ __launch_bounds__(256) void muon_prep_kernel(const MuonBatchDescs descs, const PrepArgs a) {
    __shared__ uint16_t tileT[128][64 + 2];
    __shared__ float red[2][4];
    const int tid = threadIdx.x;
    const int bat = blockIdx.y;
    const MuonMatDesc& d = descs.d[bat];
    const int64_t q = blockIdx.x;
    const bool tall = d.tall != 0;
    // Consecutive blocks take consecutive 128-column pieces of the same 64
    // parameter rows.  X coordinates: wide (i0, j0) = (r0, c0); tall (c0, r0).
    const int64_t bands = tall ? a.mp / 128 : a.np / 128;  // 128-column pieces per parameter row band
    const int64_t r0 = (q / bands) * 64, c0 = (q % bands) * 128;  // tile origin in the parameter
    const int64_t R = d.rows, C = d.cols;
    // Output: X^T (np x mp) when xt_direct, else X (mp x np).  A parameter row
    // is a row of X^T for a tall matrix (X = P^T) and a row of X for a wide
    // one; the other case goes through the LDS transpose.
    uint16_t* const out = a.xt_direct ? a.xt + bat * a.np * a.mp : a.x + bat * a.mp * a.np;
    const int64_t orows = a.xt_direct ? a.np : a.mp, ocols = a.xt_direct ? a.mp : a.np;
    const bool straight = a.xt_direct ? tall : !tall;

    // Thread tid covers 4 consecutive columns (cg) of rows rr + 8 * pass;
    // passes 0-3 are the first prep unit (rows 0-31), 4-7 the second.
    constexpr int NP = 8;
    const int cg = tid & 31, rr = tid >> 5;
    const int64_t c = c0 + cg * 4;
    const bool gb = (d.flags & MAMW_BF16_GRAD) != 0;  // gradient holds bf16
    const uint16_t* gh = reinterpret_cast<const uint16_t*>(d.grad);
    const bool vec = ((C & 3) == 0) && (reinterpret_cast<uintptr_t>(d.grad) & (gb ? 7 : 15)) == 0 &&
                     (reinterpret_cast<uintptr_t>(d.mom) & 15) == 0;
    const bool scaled = a.grad_scale != nullptr;
    const float gsc = scaled ? *a.grad_scale : 1.0f;
    const bool keep_mom = !(a.found_inf && *a.found_inf != 0.0f);
    // All passes' gradient and momentum loads are issued before any store
    // (the stores could alias later loads as far as the compiler knows, which
    // would otherwise serialise the passes).  Gradient and momentum are
    // streamed non-temporally: nothing reads them again within the step
    // (4.5-10% faster than cached accesses on the Llama-8B classes).
    float u[NP][4];
    if (vec) {
        float g[NP][4], m[NP][4];
        bool ok[NP];
#pragma unroll
        for (int pass = 0; pass < NP; ++pass) {
            const int64_t r = r0 + rr + 8 * pass;
            ok[pass] = r < R && c < C;
            if (ok[pass]) {
                const int64_t off = r * C + c;
                if (gb) {
                    const uint2 w = *reinterpret_cast<const uint2*>(gh + off);
                    g[pass][0] = bf16_to_f32(w.x & 0xffffu);
                    g[pass][1] = bf16_to_f32(w.x >> 16);
                    g[pass][2] = bf16_to_f32(w.y & 0xffffu);
                    g[pass][3] = bf16_to_f32(w.y >> 16);
                } else {
                    const f32x4_t g4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(d.grad + off));
                    g[pass][0] = g4.x;
                    g[pass][1] = g4.y;
                    g[pass][2] = g4.z;
                    g[pass][3] = g4.w;
                }
                if (scaled) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) g[pass][e] /= gsc;
                }
                const f32x4_t m4 = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(d.mom + off));
                m[pass][0] = m4.x;
                m[pass][1] = m4.y;
                m[pass][2] = m4.z;
                m[pass][3] = m4.w;
            }
        }
#pragma unroll
        for (int pass = 0; pass < NP; ++pass) {
#pragma unroll
            for (int e = 0; e < 4; ++e) u[pass][e] = 0.f;
            if (ok[pass]) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    m[pass][e] = lerp_torch(m[pass][e], g[pass][e], a.w_mom);
                    u[pass][e] = NESTEROV ? lerp_torch(g[pass][e], m[pass][e], a.w_nest) : m[pass][e];
                }
                const int64_t off = (r0 + rr + 8 * pass) * C + c;
                if (keep_mom)
                    __builtin_nontemporal_store(f32x4_t{m[pass][0], m[pass][1], m[pass][2], m[pass][3]},
                                                reinterpret_cast<f32x4_t*>(d.mom + off));
            }
        }
    } else {
#pragma unroll
        for (int pass = 0; pass < NP; ++pass) {
            const int64_t r = r0 + rr + 8 * pass;
#pragma unroll
            for (int e = 0; e < 4; ++e) u[pass][e] = 0.f;
            if (r < R && c < C) {
                const int64_t off = r * C + c;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (c + e < C) {
                        const float g0 = gb ? bf16_to_f32(gh[off + e]) : d.grad[off + e];
                        const float gv = scaled ? g0 / gsc : g0;
                        const float mv = lerp_torch(d.mom[off + e], gv, a.w_mom);
                        if (keep_mom) d.mom[off + e] = mv;
                        u[pass][e] = NESTEROV ? lerp_torch(gv, mv, a.w_nest) : mv;
                    }
                }
            }
        }
    }
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int pass = 0; pass < NP; ++pass) {
        const int rl = rr + 8 * pass;
        const int64_t r = r0 + rl;
        const uint2 pk = make_uint2(pack_bf16x2(u[pass][0], u[pass][1]), pack_bf16x2(u[pass][2], u[pass][3]));
        const uint32_t h[4] = {pk.x & 0xffffu, pk.x >> 16, pk.y & 0xffffu, pk.y >> 16};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float xb = bf16_to_f32(h[e]);
            ss[pass >> 2] += xb * xb;
        }
        if (straight) {  // parameter rows are rows of the output
            *reinterpret_cast<uint2*>(out + xoff(a.xkb, orows, ocols, r, c)) = pk;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) tileT[cg * 4 + e][rl] = uint16_t(h[e]);
        }
    }
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const float sw = wave_sum(ss[hf]);
        if ((tid & 63) == 0) red[hf][tid >> 6] = sw;
    }
    __syncthreads();
    if (tid < 2) {  // unit (32-row band 2 * (q / bands) + tid, piece q % bands)
        const int64_t unit = (2 * (q / bands) + tid) * bands + q % bands;
        a.part[bat * a.prep_tiles + unit] = (red[tid][0] + red[tid][1]) + (red[tid][2] + red[tid][3]);
    }
    if (!straight) {  // output = bf16(u)^T: row (c0 + tr), 32 consecutive elements per thread
        const int tr = tid >> 1, seg = (tid & 1) * 32;
        uint32_t w[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            w[k] = uint32_t(tileT[tr][seg + 2 * k]) | (uint32_t(tileT[tr][seg + 2 * k + 1]) << 16);
        uint4* dst = reinterpret_cast<uint4*>(out + xoff(a.xkb, orows, ocols, c0 + tr, r0 + seg));
#pragma unroll
        for (int k = 0; k < 4; ++k) dst[k] = make_uint4(w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]);
    }
}

// inv[b] = 1 / bf16(max(bf16(sqrt(sum of squares)), eps)), the value torch
// divides by in X.div_(X.norm().clamp(min=eps)) for a bf16 X.
__global__ __launch_bounds__(256) void muon_norm_kernel(const float* __restrict__ part, int64_t P,
                                                        float eps, float* __restrict__ inv) {
    __shared__ float red[4];
    const int tid = threadIdx.x, bat = blockIdx.x;
    const float* p = part + bat * P;
    // Eight independent partial sums per thread (eight loads in flight, not
    // one dependent chain), combined in a fixed order.
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t i = tid;
    for (; i + 7 * 256 < P; i += 8 * 256) {
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] += p[i + u * 256];
    }
    for (; i < P; i += 256) a[0] += p[i];
    float s = ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    if (tid == 0) {
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float nrm = bf16_to_f32(f32_to_bf16(sqrtf(tot)));
        const float clamped = bf16_to_f32(f32_to_bf16(fmaxf(nrm, eps)));
        inv[bat] = 1.0f / clamped;
    }
}

// XT_ONLY (xt_direct): XT = bf16(XT * inv[b]) in place, a plain stream of
// 16-byte pieces, four per thread (all loads before the stores), 8192
// elements per block; NT: non-temporal loads and stores (for a group's X^T
// larger than the memory-side cache: 8% faster there, 15% slower on groups it
// holds).
// Otherwise (the row-major workspace): XT = bf16(X * inv[b])^T and
// X <- bf16(X * inv[b]) in place, one 128 x 64 tile of X per block (two prep
// units), 16-byte global accesses throughout.  Each thread scales a 4 x 8
// block (rows 4rq..4rq+3, columns 8cg..8cg+7) and writes its 8 columns to the
// LDS transpose as 8-byte runs of 4 rows.  tileT row c (X column c) holds 128
// elements as 16 chunks of 16 bytes, chunk k stored at k ^ scale_swz(c): the
// 8-byte column writes of 32 lanes and the 16-byte row reads of 16 lanes each
// touch every bank once (2-byte writes into a padded tile measured 85% of the
// kernel's LDS cycles in bank conflicts).
__device__ __forceinline__ int scale_swz(int c) { return ((c >> 3) << 1) ^ (c & 3); }

template <bool XT_ONLY, bool NT = false>
__global__ __launch_bounds__(256) void muon_scale_kernel(const PrepArgs a, const float* __restrict__ inv) {
    if constexpr (XT_ONLY) {
        const int bat = blockIdx.y;
        uint4* xt = reinterpret_cast<uint4*>(a.xt + bat * a.np * a.mp) + int64_t(blockIdx.x) * 1024 + threadIdx.x;
        const float sc = inv[bat];
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        uint4 w[4];
        if constexpr (NT) {
#pragma unroll
            for (int p = 0; p < 4; ++p)
                w[p] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(xt + 256 * p)));
#pragma unroll
            for (int p = 0; p < 4; ++p)
                __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, scale_bf16x8(w[p], sc)),
                                            reinterpret_cast<u32x4_t*>(xt + 256 * p));
        } else {
#pragma unroll
            for (int p = 0; p < 4; ++p) w[p] = xt[256 * p];
#pragma unroll
            for (int p = 0; p < 4; ++p) xt[256 * p] = scale_bf16x8(w[p], sc);
        }
        return;
    }
    __shared__ uint4 tileT[64][16];
    const int tid = threadIdx.x, bat = blockIdx.y;
    const int64_t q = blockIdx.x;
    const int64_t i0 = (q / a.tiles_j) * 128, j0 = (q % a.tiles_j) * 64;
    uint16_t* X = a.x + bat * a.mp * a.np;
    uint16_t* XT = a.xt + bat * a.np * a.mp;
    const float s = inv[bat];
    const int cg = tid & 7, rq = tid >> 3;
    uint4 v[4];  // all four loads before the in-place stores
#pragma unroll
    for (int p = 0; p < 4; ++p)
        v[p] = *reinterpret_cast<const uint4*>(X + xoff(a.xkb, a.mp, a.np, i0 + 4 * rq + p, j0 + cg * 8));
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        v[p] = scale_bf16x8(v[p], s);
        *reinterpret_cast<uint4*>(X + xoff(a.xkb, a.mp, a.np, i0 + 4 * rq + p, j0 + cg * 8)) = v[p];
    }
    uint2* t2 = reinterpret_cast<uint2*>(&tileT[0][0]);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint32_t w[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t x2 = (e >> 1) == 0 ? v[p].x : (e >> 1) == 1 ? v[p].y : (e >> 1) == 2 ? v[p].z : v[p].w;
            w[p] = (e & 1) ? (x2 >> 16) : (x2 & 0xffffu);
        }
        const int c = cg * 8 + e;
        const int unit = (((rq >> 1) ^ scale_swz(c)) << 1) | (rq & 1);
        t2[c * 32 + unit] = make_uint2(w[0] | (w[1] << 16), w[2] | (w[3] << 16));
    }
    __syncthreads();
    // XT row (j0 + tr), elements i0 + 32 * sq .. + 31: 64 contiguous bytes per thread.
    const int tr = tid >> 2, sq = tid & 3;
    uint4* dst = reinterpret_cast<uint4*>(XT + xoff(a.xkb, a.np, a.mp, j0 + tr, i0 + 32 * sq));
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[k] = tileT[tr][(4 * sq + k) ^ scale_swz(tr)];
}

// ns_steps == 0: the update is the normalised X itself (read from X^T).
__global__ __launch_bounds__(256) void muon_apply0_kernel(const MuonBatchDescs descs, const PrepArgs a, float keep) {
    if (a.found_inf && *a.found_inf != 0.0f) return;  // skipped gradient-scaler step
    const int bat = blockIdx.y;
    const MuonMatDesc& d = descs.d[bat];
    const uint16_t* XT = a.xt + bat * a.mp * a.np;
    const int64_t total = d.rows * d.cols;
    for (int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x; e < total; e += int64_t(gridDim.x) * 256) {
        const int64_t r = e / d.cols, c = e % d.cols;
        // X[i][j] = XT[j][i] with (i, j) = (c, r) for a tall parameter, (r, c) otherwise
        const float u = bf16_to_f32(d.tall ? XT[xoff(a.xkb, a.np, a.mp, r, c)] : XT[xoff(a.xkb, a.np, a.mp, c, r)]);
        if (d.flags & MAMW_BF16_PARAM) {
            uint16_t* ph = reinterpret_cast<uint16_t*>(d.param);
            ph[e] = uint16_t(f32_to_bf16(__builtin_fmaf(-d.slr, u, bf16_to_f32(ph[e]) * keep)));
        } else {
            d.param[e] = __builtin_fmaf(-d.slr, u, d.param[e] * keep);
        }
        if (d.upd) d.upd[e] = u;
    }
}

// ---------------------------------------------------------------------------
// MFMA GEMM: C[i][j] = sum_k Aop[i][k] * Bop[j][k]  (bf16 in, fp32 accumulate).
//
// Block tile BM x BM, 4 waves in a 2 x 2 layout, each wave a (BM/2) x (BM/2)
// sub-tile built from v_mfma_f32_32x32x16_bf16 (accumulators in AGPRs).  K
// advances in steps of 64 through two LDS buffers filled straight from global
// memory by buffer_load_dwordx4 ... lds (no VGPR staging; one buffer resource
// per operand tile, so a lane needs a single 32-bit offset per operand).
//
// A step is four 16-wide k slices of NMF MFMAs each.  Every slice issues its
// MFMAs one at a time with the next slice's fragment reads woven in between
// (sched_barrier keeps that order), so the matrix pipe never waits for an
// address computation.  The DMA of a step is split in two halves: the first
// goes out in the last slice of the step two ahead, the second in the first
// slice of the next step, one load per two MFMAs.  Spreading the loads keeps
// the per-CU queue of outstanding L2 requests busy without the load issue
// stalling the MFMAs behind it (one 16-load burst per step measured 5-9%
// slower).  The block barrier sits before the last slice: the MFMAs of that
// slice run from registers while the barrier releases the buffer just read,
// and the next step's first fragments are read under them.  LDS rows
// are 128 bytes with the 16-byte chunk index XOR-swizzled (lds_chunk), so
// fragment reads are bank-conflict free.

struct GemmArgs {
    const uint16_t* aop;  // A operand, batch 0 (rows i)
    const uint16_t* bop;  // B operand, batch 0 (rows j)
    int64_t a_bs, b_bs;   // batch strides (elements)
    int64_t lda, ldb;
    int K;                // multiple of 64
    int tiles_m, tiles_n;
    int tiles_per_matrix; // tiles of one matrix in the launch (upper triangle when symmetric)
    uint16_t* c;          // GRAM/POLY: symmetric output; UPDATE: X (NULL: X^T only)
    int64_t c_bs, ldc;
    uint16_t* ct;         // UPDATE: X^T (may be NULL in the standalone entry)
    int64_t ct_bs, ldct;
    const uint16_t* src;  // POLY: A;  UPDATE/APPLY: X^T (read transposed as X)
    int64_t src_bs, lds;
    float alpha;          // coefficient on the accumulator
    float beta;           // coefficient on src
    float keep;           // APPLY: 1 - lr * weight_decay
    int64_t m, n;         // APPLY: valid extent of X
    int xkb;              // operands, coefficient and outputs k-blocked (xoff)
    const float* found_inf;  // APPLY: a non-zero *found_inf (skipped gradient-scaler step) writes nothing
    int kmajor;           // GRAM, k-blocked: operands are X^T (lda = its rows), read k-major
    int lower;            // GRAM/POLY, k-blocked: write only the lower triangle (the transposed orientation)
    int a_low;            // POLY/UPDATE/APPLY, k-blocked: the symmetric operand (A; B) holds only its lower triangle
};

// Launch block -> (matrix, tile row, tile col).
//
// The operand bytes a block needs per k step are fixed by the tile, so what
// sets the speed is where they come from.  Blocks are dealt to the 8 XCDs
// round-robin, 32 CUs each.  The remap gives every XCD, in each round of
// 8 x 32 blocks, 32 consecutive logical tiles (a compact patch of one matrix
// whose tiles share operand rows in that XCD's L2), and gives the 8 XCDs
// neighbouring patches, so the round's operands are one matrix's worth and stay
// in the memory-side cache.  An incomplete last round (all of a grid smaller
// than 8 x 32) is cut into 8 contiguous ranges, one per XCD.  Logical order
// within a matrix: groups of GM tile rows, column by column (symmetric
// products: only the tiles with ti <= tj).  GM = 4 for 256-wide tiles; 8 for
// 128-wide tiles, whose rounds hold twice the blocks (two per CU), so that an
// XCD's share of a small matrix (m = 768: all six tile rows) reads each X^T
// panel once (GPT-2's updates 4% faster than with groups of 4, Grams 1%).
constexpr int kXcds = 8;
constexpr int kXcdSlots = 32;

template <bool SYM, int kGroupM>
__device__ __forceinline__ void decode_tile(const GemmArgs& g, int& bat, int& ti, int& tj) {
    const int L = blockIdx.x, total = gridDim.x;
    const int full = (total / (kXcds * kXcdSlots)) * (kXcds * kXcdSlots);
    const int xcd = L % kXcds, j = L / kXcds;
    const int rem = total - full, q = rem / kXcds, r = rem % kXcds;  // the last round: XCD x gets q or q+1
    const int logical = L < full ? ((j / kXcdSlots) * kXcds + xcd) * kXcdSlots + j % kXcdSlots
                                 : full + xcd * q + min(xcd, r) + (L - full) / kXcds;
    bat = logical / g.tiles_per_matrix;
    int t = logical - bat * g.tiles_per_matrix;
    const int T = g.tiles_m;
    if (SYM) {
        // Group of rows [first, first+gs): a triangle (column first+c holds
        // rows first..first+c), then full columns of gs rows.
        int first = 0, gs = min(kGroupM, T);
        for (;;) {
            const int gtiles = gs * (gs + 1) / 2 + (T - first - gs) * gs;
            if (t < gtiles) break;
            t -= gtiles;
            first += gs;
            gs = min(kGroupM, T - first);
        }
        const int tri = gs * (gs + 1) / 2;
        if (t < tri) {
            int c = 0;
            while ((c + 1) * (c + 2) / 2 <= t) ++c;
            tj = first + c;
            ti = first + t - c * (c + 1) / 2;
        } else {
            t -= tri;
            tj = first + gs + t / gs;
            ti = first + t % gs;
        }
    } else {
        const int width = kGroupM * g.tiles_n;
        const int group = t / width, first = group * kGroupM;
        const int gsize = min(T - first, kGroupM);
        const int w = t - group * width;
        ti = first + w % gsize;
        tj = w / gsize;
    }
}

// Physical 16-byte chunk of logical chunk `ch` (0..7) in LDS row `row` (64
// bf16 per row).  XOR-ing with (row & 7) ^ ((row >> 3) & 1) makes any 16
// consecutive rows at one logical chunk land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_chunk(int row, int ch) { return ch ^ (row & 7) ^ ((row >> 3) & 1); }

// Buffer resource over `bytes` bytes from `base` (raw buffer, 32-bit dwords).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes), 0x00020000);
}

// APPLY on up to 8 consecutive elements of one parameter row, in two halves so
// that a caller can issue the parameter loads of several pieces before any
// store (to the compiler a store could alias a later load, which would
// otherwise serialise the pieces behind the HBM latency): with u the bf16
// update values in w, param[idx + e] = param*keep - slr*u (and upd = u) for
// e < nv.  apply_begin loads the parameter when the piece is 8 elements on
// 16-byte boundaries (the common case); the caller then sets w, and
// apply_end finishes the piece, or does it element by element otherwise.
struct ApplyPiece {
    uint4 w;       // bf16 update values
    uint4 p0, p1;  // fp32 parameter: two float4 bit patterns; bf16 parameter: p0
    int64_t idx;   // parameter element index of the first value
    int nv;        // values to apply (0..8)
    bool fast;     // p0 / p1 hold the loaded parameter
};

// NT: non-temporal parameter accesses (the parameter rows of a tall matrix,
// written from whole tile columns: measured 4% faster on the 14336 x 4096
// Llama-8B matrices; the wide matrices' row pieces measured 1.5% slower so).
typedef unsigned int nt_u32x4_t __attribute__((ext_vector_type(4)));
template <bool NT = false>
__device__ __forceinline__ uint4 load_u4(const uint4* q) {
    if constexpr (NT) {
        const nt_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const nt_u32x4_t*>(q));
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    return *q;
}
template <bool NT = false>
__device__ __forceinline__ void store_u4(uint4* q, uint4 w) {
    if constexpr (NT)
        __builtin_nontemporal_store(nt_u32x4_t{w.x, w.y, w.z, w.w}, reinterpret_cast<nt_u32x4_t*>(q));
    else
        *q = w;
}

template <bool NT = false>
__device__ __forceinline__ void apply_begin(const MuonMatDesc& d, ApplyPiece& a, int64_t prow, int64_t pcol,
                                            int64_t cap, int64_t left) {
    const int64_t nv = cap < left ? cap : left;
    a.nv = nv > 0 ? int(nv) : 0;
    a.idx = prow * d.cols + pcol;
    const bool bf = (d.flags & MAMW_BF16_PARAM) != 0;
    const uintptr_t pa = bf ? reinterpret_cast<uintptr_t>(reinterpret_cast<uint16_t*>(d.param) + a.idx)
                            : reinterpret_cast<uintptr_t>(d.param + a.idx);
    const uintptr_t ua = d.upd ? reinterpret_cast<uintptr_t>(d.upd + a.idx) : 0;
    a.fast = a.nv == 8 && ((pa | ua) & 15) == 0;
    if (a.fast) {
        const uint4* q = reinterpret_cast<const uint4*>(pa);
        a.p0 = load_u4<NT>(q);
        if (!bf) a.p1 = load_u4<NT>(q + 1);
    }
}

// apply_begin through a buffer resource `rp` over the parameter elements from
// element `base` on: every piece issues exactly its loads (two 16-byte loads
// for an fp32 parameter, one for bf16), those of a piece that apply_end will
// not read whole (ragged or unaligned, or outside the matrix) at an offset past
// the resource's end, which reads zeros without touching memory.  A caller can
// then wait for older loads with a fixed vmcnt while these stay in flight.
template <bool NT = false>
__device__ __forceinline__ void apply_begin_buf(const MuonMatDesc& d, ApplyPiece& a, int64_t prow, int64_t pcol,
                                                int64_t cap, int64_t left, __amdgpu_buffer_rsrc_t rp,
                                                int64_t base) {
    const int64_t nv = cap < left ? cap : left;
    a.nv = nv > 0 ? int(nv) : 0;
    a.idx = prow * d.cols + pcol;
    const bool bf = (d.flags & MAMW_BF16_PARAM) != 0;
    const uintptr_t pa = bf ? reinterpret_cast<uintptr_t>(reinterpret_cast<uint16_t*>(d.param) + a.idx)
                            : reinterpret_cast<uintptr_t>(d.param + a.idx);
    const uintptr_t ua = d.upd ? reinterpret_cast<uintptr_t>(d.upd + a.idx) : 0;
    a.fast = a.nv == 8 && ((pa | ua) & 15) == 0;
    const int off = a.fast ? int((a.idx - base) * (bf ? 2 : 4)) : 0x7FFFFF00;
    typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t v0 = __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, NT ? 2 : 0);
    a.p0 = make_uint4(v0.x, v0.y, v0.z, v0.w);
    if (!bf) {
        const u32x4_t v1 = __builtin_amdgcn_raw_buffer_load_b128(rp, off + 16, 0, NT ? 2 : 0);
        a.p1 = make_uint4(v1.x, v1.y, v1.z, v1.w);
    }
}

template <bool NT = false>
__device__ __forceinline__ void apply_end(const MuonMatDesc& d, const ApplyPiece& a, float keep) {
    if (a.nv == 0) return;
    const uint32_t ww[4] = {a.w.x, a.w.y, a.w.z, a.w.w};
    float u[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        u[2 * j] = bf16_to_f32(ww[j] & 0xffffu);
        u[2 * j + 1] = bf16_to_f32(ww[j] >> 16);
    }
    float* up = d.upd ? d.upd + a.idx : nullptr;
    if (a.fast) {
        if (d.flags & MAMW_BF16_PARAM) {  // bf16 parameter: fp32 arithmetic, rounded back to nearest-even
            const uint32_t pv[4] = {a.p0.x, a.p0.y, a.p0.z, a.p0.w};
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                o[j] = pack_bf16x2(__builtin_fmaf(-d.slr, u[2 * j], bf16_to_f32(pv[j] & 0xffffu) * keep),
                                   __builtin_fmaf(-d.slr, u[2 * j + 1], bf16_to_f32(pv[j] >> 16) * keep));
            uint16_t* ph = reinterpret_cast<uint16_t*>(d.param) + a.idx;
            store_u4<NT>(reinterpret_cast<uint4*>(ph), make_uint4(o[0], o[1], o[2], o[3]));
        } else {
            const uint32_t pv[8] = {a.p0.x, a.p0.y, a.p0.z, a.p0.w, a.p1.x, a.p1.y, a.p1.z, a.p1.w};
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = __builtin_fmaf(-d.slr, u[j], __uint_as_float(pv[j]) * keep);
            uint4* p = reinterpret_cast<uint4*>(d.param + a.idx);
            store_u4<NT>(p, make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                       __float_as_uint(o[3])));
            store_u4<NT>(p + 1, make_uint4(__float_as_uint(o[4]), __float_as_uint(o[5]), __float_as_uint(o[6]),
                                           __float_as_uint(o[7])));
        }
        if (up) {
            reinterpret_cast<float4*>(up)[0] = make_float4(u[0], u[1], u[2], u[3]);
            reinterpret_cast<float4*>(up)[1] = make_float4(u[4], u[5], u[6], u[7]);
        }
        return;
    }
    if (d.flags & MAMW_BF16_PARAM) {
        uint16_t* ph = reinterpret_cast<uint16_t*>(d.param) + a.idx;
        for (int e = 0; e < a.nv; ++e) {
            ph[e] = uint16_t(f32_to_bf16(__builtin_fmaf(-d.slr, u[e], bf16_to_f32(ph[e]) * keep)));
            if (up) up[e] = u[e];
        }
    } else {
        float* p = d.param + a.idx;
        for (int e = 0; e < a.nv; ++e) {
            p[e] = __builtin_fmaf(-d.slr, u[e], p[e] * keep);
            if (up) up[e] = u[e];
        }
    }
}

// BM x BN tiles: BM rows of the A operand (i), BN rows of the B operand (j).
// 256 x 256: one workgroup per CU.  128 x 128 and 128 x 192 (the updates of
// matrices with m < 1024, n a multiple of 192): two workgroups per CU (64 and
// 80 KB of LDS, at most 256 registers per lane each).
template <int BM, int MODE, bool KB, bool KM = false, bool LOW = false, int BN = BM>
__global__ __launch_bounds__(kGemmThreads, BM == 128 ? 2 : 1) void ns_gemm_kernel(const GemmArgs g,
                                                                                 const MuonBatchDescs descs) {
    static_assert(!KM || (KB && MODE == MODE_GRAM), "k-major operands: the k-blocked Gram only");
    static_assert(!LOW || (KB && MODE != MODE_GRAM), "lower-triangle operands: polynomial and updates, k-blocked");
    static_assert(BN == BM || (KB && (MODE == MODE_UPDATE || MODE == MODE_APPLY) && BM == 128 && BN == 192),
                  "rectangular tiles: the k-blocked updates, 128 x 192");
    // LOW: the symmetric operand (A of the polynomial, both sides; B of the
    // updates, side A) holds only its lower triangle of BM x BM blocks.
    constexpr bool LOWA = LOW, LOWB = LOW && MODE == MODE_POLY;
    constexpr int WTM = BM / 2, WTN = BN / 2;  // wave tile (2 x 2 waves)
    constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 fragments per wave tile edge
    constexpr int NMF = FM * FN;            // MFMAs per 16-wide k slice
    constexpr int LA = BM / 32, LB = BN / 32;  // DMA loads per wave per step (8 rows each) of the A / B operand
    constexpr int RPM = (FM + FN + NMF - 1) / NMF;   // fragment reads woven in per MFMA
    constexpr int LPM = (LA + LB + NMF - 1) / NMF;  // coefficient-tile DMA loads woven in per MFMA
    constexpr int STAGE = (BM + BN) * kBK;  // bf16 elements per LDS stage
    constexpr bool SYM = (MODE == MODE_GRAM || MODE == MODE_POLY);
    __shared__ uint4 smem_v[2 * STAGE / 8];
    uint16_t* smem = reinterpret_cast<uint16_t*>(smem_v);

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    if constexpr (MODE == MODE_APPLY) {
        if (g.found_inf && *g.found_inf != 0.0f) return;  // uniform per launch: the whole block leaves
    }
    int bat, ti, tj;
    decode_tile<SYM, BM == 128 ? 8 : 4>(g, bat, ti, tj);
    // Uniform by construction; pinned to scalar registers so that every
    // buffer resource derived from them is one (a resource the compiler
    // cannot prove uniform turns each load into a loop over the lanes).
    bat = __builtin_amdgcn_readfirstlane(bat);
    ti = __builtin_amdgcn_readfirstlane(ti);
    tj = __builtin_amdgcn_readfirstlane(tj);
    // Operand rows of the tile: row-major (row stride ld), or k-blocked (KB:
    // row stride 64 inside a 64-wide panel, panel stride rows*64).  The buffer
    // resource spans the tile's rows up to column K.
    constexpr bool KBOP = KB;
    const int64_t rows_a = int64_t(g.tiles_m) * BM, rows_b = int64_t(g.tiles_n) * BN;
    // KM: the operand is X^T (g.lda rows, k-blocked), and the tile's BM
    // columns of it are BM/64 whole panels of g.lda rows x 128 bytes.
    const uint16_t* Ag = KM ? g.aop + bat * g.a_bs + int64_t(ti) * (BM / 64) * g.lda * 64
                            : g.aop + bat * g.a_bs + int64_t(ti) * BM * (KBOP ? 64 : g.lda);
    const uint16_t* Bg = KM ? g.bop + bat * g.b_bs + int64_t(tj) * (BN / 64) * g.ldb * 64
                            : g.bop + bat * g.b_bs + int64_t(tj) * BN * (KBOP ? 64 : g.ldb);
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(Ag, KM ? (BM / 64) * g.lda * 128
                         : KBOP ? ((g.K / 64 - 1) * rows_a + BM) * 128 : ((BM - 1) * g.lda + g.K) * 2);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(Bg, KM ? (BN / 64) * g.ldb * 128
                         : KBOP ? ((g.K / 64 - 1) * rows_b + BN) * 128 : ((BN - 1) * g.ldb + g.K) * 2);
    const int pk2 = int(g.lda) * 128;  // KM: bytes per panel
    const int pa2 = int(rows_a) * 128, pb2 = int(rows_b) * 128;  // KBOP: bytes per k-step panel
    // A lower-triangle operand (LOWA / LOWB): the side's rows r (ti or tj)
    // read block (r, kb) row-major while kb < r and block (kb, r) k-major
    // after (rows k, columns r: S[k][r] = S[r][k]).  The diagonal block is
    // stored whole and exactly symmetric, so it can be read either way:
    // k-major for r > 0, row-major for r = 0.  The switch step
    // ksw = max(r, 1) BM/64 then leaves at least BM/64 steps on each side (the
    // host uses these layouts only with two or more block rows).  Loads pick
    // their layout arithmetically from the step they load (no branches);
    // fragment reads follow the loop segment they are in.
    const int ksw_a = LOWA ? max(ti, 1) * (BM / 64) : 1 << 30;
    const int ksw_b = LOWB ? max(tj, 1) * (BN / 64) : 1 << 30;
    const __amdgpu_buffer_rsrc_t ra_low = make_rsrc(g.aop + bat * g.a_bs, LOWA ? rows_a * rows_a * 2 : 0);
    const __amdgpu_buffer_rsrc_t rb_low = make_rsrc(g.bop + bat * g.b_bs, LOWB ? rows_b * rows_b * 2 : 0);
    const int a_km_off = ti * (BM / 64) * pa2;  // tile offsets (bytes): A k-major, B in each layout
    const int b_kb_off = tj * BN * 128, b_km_off = tj * (BN / 64) * pb2;

    // Load i (0..LOADS-1) of an operand fills rows row0 = wave*BM/4 + 8i ..
    // row0+7: lane l lands at physical chunk l&7 of row row0 + l/8, which holds
    // logical chunk (l&7) ^ (l/8) ^ (i&1)  (lds_chunk with row0 a multiple of 8).
    const int lrow = lane >> 3;
    const int lda2 = KBOP ? 128 : int(g.lda) * 2, ldb2 = KBOP ? 128 : int(g.ldb) * 2;
    const int va0 = lrow * lda2 + (((lane & 7) ^ lrow) << 4), va1 = lrow * lda2 + (((lane & 7) ^ lrow ^ 1) << 4);
    const int vb0 = lrow * ldb2 + (((lane & 7) ^ lrow) << 4), vb1 = lrow * ldb2 + (((lane & 7) ^ lrow ^ 1) << 4);
    // KM: an operand's stage is BM/64 panels of 64 k rows x 128 bytes, 1-KB
    // block lc holding k rows (lc%8)*8.. of panel lc/8; a k row stores logical
    // chunk c at physical chunk c ^ kswz, kswz = 4 for rows 2,3 (mod 4), so the
    // transpose reads below (4 rows x 64 bytes per 32 lanes) are conflict free.
    const int vk = lrow * 128 + (((lane & 7) ^ (((lrow >> 1) & 1) << 2)) << 4);
    // DMA number i: operand A for i < LA, else B.
    // Both layouts put a load's 1 KB at the same LDS bytes (lc * 512 ==
    // row0 * kBK), so a lower-triangle side only switches the source address.
    // la (std::bool_constant, LOWA): the A rows of the step loaded are k-major;
    // every call site knows it.  The B side's switch step depends on the tile
    // pair, so LOWB picks the layout arithmetically from the step loaded.
    auto load1 = [&](int i, int k0, int buf, auto la) __attribute__((always_inline)) {
        const int ii = i < LA ? i : i - LA, row0 = wave * ((i < LA ? BM : BN) / 4) + ii * 8;
        if constexpr (LOWA && decltype(la)::value) {
            if (i < LA) {
                const int lc = wave * LA + ii;
                uint16_t* dst = smem + buf * STAGE + lc * 512;
                const int soff =
                    __builtin_amdgcn_readfirstlane(a_km_off + (lc >> 3) * pa2 + (k0 + (lc & 7) * 8) * 128);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_low, (lds_ptr_t)dst, 16, vk, soff, 0, 0);
                return;
            }
        }
        if constexpr (LOWB) {
            if (i >= LA) {
                const int lc = wave * LB + ii;
                uint16_t* dst = smem + buf * STAGE + BM * kBK + lc * 512;
                const int f = 1 + ((k0 - ksw_b * kBK) >> 31);  // 1: k-major
                const int s_rm = b_kb_off + row0 * 128 + (k0 >> 6) * pb2;
                const int s_km = b_km_off + (lc >> 3) * pb2 + (k0 + (lc & 7) * 8) * 128;
                const int soff = __builtin_amdgcn_readfirstlane(s_rm + f * (s_km - s_rm));
                const int v_rm = (ii & 1) ? vb1 : vb0;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_low, (lds_ptr_t)dst, 16, v_rm + f * (vk - v_rm), soff, 0,
                                                         0);
                return;
            }
        }
        if constexpr (KM) {
            const int lc = wave * (i < LA ? LA : LB) + ii;
            uint16_t* dst = smem + buf * STAGE + (i < LA ? 0 : BM * kBK) + lc * 512;
            const int soff = (lc >> 3) * pk2 + (k0 + (lc & 7) * 8) * 128;
            if (i < LA)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)dst, 16, vk, soff, 0, 0);
            else
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)dst, 16, vk, soff, 0, 0);
            return;
        }
        uint16_t* dst = smem + buf * STAGE + (i < LA ? 0 : BM * kBK) + row0 * kBK;
        if (i < LA)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)dst, 16, (ii & 1) ? va1 : va0,
                                                     row0 * lda2 + (KBOP ? (k0 >> 6) * pa2 : k0 * 2), 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)dst, 16, (ii & 1) ? vb1 : vb0,
                                                     row0 * ldb2 + (KBOP ? (k0 >> 6) * pb2 : k0 * 2), 0, 0);
    };
    // KM fragment: two transpose reads of 4 k rows each.  In a 16-lane group
    // lane s names k row (s/4) and columns 4(s%4).. of the group's 16 columns,
    // so lane i receives column i at 4 consecutive k; lanes 16-31 take the next
    // 16 columns, lanes 32-63 the rows 8 below.  km_o[b] is the lane's element
    // offset inside its panel's k slice for a fragment at column 32b of it.
    // km_base[side][b]: the lane's LDS byte address in stage buffer 0 for a
    // fragment at column 32b of the first panel of this wave's rows (side 0,
    // wm) or columns (side 1, wn); the rest is an immediate offset.
    uint32_t km_base[2][2];
    {
        const int s = lane & 15, kx = ((s >> 3) & 1) << 2, lcl = 2 * ((lane >> 4) & 1) + ((s & 3) >> 1);
        const int rowo = ((lane >> 5) * 8 + (s >> 2)) * 64 + (s & 1) * 4;
        const int km_o[2] = {rowo + ((kx | lcl) << 3), rowo + (((4 ^ kx) | lcl) << 3)};
        const uint32_t s0 = lds_addr(smem);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            km_base[0][b] = s0 + ((wm * WTM) >> 6) * 8192 + km_o[b] * 2;
            km_base[1][b] = s0 + BM * kBK * 2 + ((wn * WTN) >> 6) * 8192 + km_o[b] * 2;
        }
    }
    // Fragment read j of slice ks, in the order the MFMAs first use them
    // (a-major): fa0, fb0 .. fb[FN-1], fa1 .. fa[FM-1].
    // kma, kmb: the A / B side of this step is read k-major (lower-triangle
    // operands past their switch step); std::bool_constant, so each call
    // site compiles one path.
    auto read1 = [&](bf16x8_t (&fa)[FM], bf16x8_t (&fb)[FN], int buf, int ks, int j, auto kma, auto kmb)
                     __attribute__((always_inline)) {
        const uint16_t* base = smem + buf * STAGE;
        const int ch = ks * 2 + (lane >> 5);
        const bool isa = (j == 0) || (j > FN);
        const int f = j == 0 ? 0 : (j <= FN ? j - 1 : j - FN);
        if constexpr (!KM && (decltype(kma)::value || decltype(kmb)::value)) {
            if (isa ? decltype(kma)::value : decltype(kmb)::value) {
                const uint32_t q = km_base[isa ? 0 : 1][f & 1] + uint32_t(buf) * (STAGE * 2);
                const int off = (f >> 1) * 8192 + ks * 2048;
                const uint2 lo = lds_read_tr16_untracked(q, off), hi = lds_read_tr16_untracked(q, off + 512);
                const bf16x8_t v = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                if (isa)
                    fa[f] = v;
                else
                    fb[f] = v;
                return;
            }
        }
        if constexpr (KM) {
            // column 32f of the wave's range: panel f/2, column half f%2
            const uint32_t q = km_base[isa ? 0 : 1][f & 1] + uint32_t(buf) * (STAGE * 2);
            const int off = (f >> 1) * 8192 + ks * 2048;
            const uint2 lo = lds_read_tr16_untracked(q, off), hi = lds_read_tr16_untracked(q, off + 512);
            const bf16x8_t v = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
            if (isa)
                fa[f] = v;
            else
                fb[f] = v;
            return;
        }
        if (isa) {
            const int r = wm * WTM + f * 32 + (lane & 31);
            fa[f] = *reinterpret_cast<const bf16x8_t*>(base + r * kBK + (lds_chunk(r, ch) << 3));
        } else {
            const int r = wn * WTN + f * 32 + (lane & 31);
            fb[f] = *reinterpret_cast<const bf16x8_t*>(base + BM * kBK + r * kBK + (lds_chunk(r, ch) << 3));
        }
    };

    f32x16_t acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.f;
    // Epilogue coefficient tile (POLY: A; UPDATE/APPLY: X^T), stored
    // transposed in LDS as TT[x][y] = src[tj*BN + x][ti*BM + y] (A is
    // symmetric; X^T holds X transposed), in 1-KB DMA blocks: block b fills TT
    // rows b*RPI .. b*RPI+RPI-1.  TT row x holds 16-byte chunks of BM/8 y
    // values, logical chunk c at physical chunk c ^ (x ^ x>>3) (mod BM/8).
    constexpr int NCH = BM / 8;                   // 16-byte chunks per TT row
    constexpr int RPI = 64 / NCH;                 // TT rows per 1-KB block
    constexpr int NSB = BN / RPI;                 // blocks of the whole tile
    constexpr int NPRE = STAGE * 2 / 1024;        // blocks in stage buffer 0 (all of TT when BM = BN = 128)
    static_assert(NPRE == 4 * (LA + LB) && NPRE <= NSB, "prefetch blocks map onto the DMA slots of one step");
    // Rows of the coefficient matrix and of the transposed-orientation output
    // (A or B: mp; X^T: np), which address their k-blocked panels.
    const int64_t rows_t = int64_t(g.tiles_n) * BN;
    const uint16_t* S = MODE == MODE_GRAM ? g.aop  // (unused)
                      : KB ? g.src + bat * g.src_bs + (int64_t(ti) * (BM / 64) * rows_t + int64_t(tj) * BN) * 64
                           : g.src + bat * g.src_bs + int64_t(tj) * BN * g.lds + int64_t(ti) * BM;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(S, MODE == MODE_GRAM ? 0
                                                   : KB ? ((BM / 64 - 1) * rows_t + BN) * 128
                                                        : ((BN - 1) * g.lds + BM) * 2);
    const int lds2 = MODE == MODE_GRAM ? 0 : KB ? 128 : int(g.lds) * 2;  // bytes between TT rows' sources
    const int pnl2 = int(rows_t) * 128;                                   // KB: bytes per 64-column panel
    auto src_load = [&](int b) __attribute__((always_inline)) {
        const int x0 = b * RPI, x = x0 + lane / NCH;
        const int c = ((lane % NCH) ^ x ^ (x >> 3)) & (NCH - 1);  // logical chunk at physical lane % NCH
        const int coff = KB ? (c >> 3) * pnl2 + (c & 7) * 16 : c * 16;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(smem + x0 * BM), 16, (lane / NCH) * lds2 + coff,
                                                 x0 * lds2, 0, 0);
    };

    // One slice: MFMAs on (ca, cb); reads of the next slice into (na, nb) when
    // `reads`; per `loads`, DMA loads [llo, lhi) of step k0/kBK into buffer
    // lbuf (1) or this wave's share of the coefficient blocks that fit in stage
    // buffer 0 (2).  All arguments are compile-time constants at every call, so
    // the body has no branches.
    // kma, kmb: this step's fragments are read k-major on the A / B side; then
    // (ca, cb) came from untracked reads, which the first MFMA waits for.
    auto slice = [&](const bf16x8_t (&ca)[FM], const bf16x8_t (&cb)[FN], bf16x8_t (&na)[FM], bf16x8_t (&nb)[FN],
                     bool reads, int rbuf, int rks, int loads, int k0, int lbuf, int llo, int lhi, auto kma,
                     auto kmb, auto la) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            if constexpr (KM || decltype(kma)::value || decltype(kmb)::value) {
                if (i == 0) {
                    // (ca, cb) came from the untracked reads of the previous
                    // slice: all of them are complete before its first MFMA
                    // (waiting per MFMA for just its fragments, or spreading
                    // the reads over all MFMAs, measured slower).
                    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            acc[i / FN][i % FN] =
                __builtin_amdgcn_mfma_f32_32x32x16_bf16(ca[i / FN], cb[i % FN], acc[i / FN][i % FN], 0, 0, 0);
#pragma unroll
            for (int r = 0; r < RPM; ++r)
                if (reads && i * RPM + r < FM + FN) read1(na, nb, rbuf, rks, i * RPM + r, kma, kmb);
#pragma unroll
            for (int l = 0; l < LPM; ++l)
                if (loads == 2 && i * LPM + l < LA + LB) src_load(wave * (LA + LB) + i * LPM + l);
            if (loads == 1) {
                const int nl = lhi - llo, j0 = llo + (i * nl) / NMF, j1 = llo + ((i + 1) * nl) / NMF;
#pragma unroll
                for (int j = j0; j < j1; ++j) load1(j, k0, lbuf, la);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    const int KT = g.K / kBK;
    // DMA loads per step; the half issued two steps ahead (every A load and
    // the first B loads: the second half holds no A load).
    constexpr int NL = LA + LB, LH = NL / 2;
    static_assert(LH >= LA, "the second half of a step's loads is B only");
#pragma unroll
    for (int i = 0; i < NL; ++i) load1(i, 0, 0, std::false_type{});  // steps 0, 1: below any switch
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    if (KT > 1) {
#pragma unroll
        for (int i = 0; i < LH; ++i) load1(i, kBK, 1, std::false_type{});
    }
    bf16x8_t fa0[FM], fb0[FN], fa1[FM], fb1[FN];
    if constexpr (!LOW) {  // LOW: each loop segment reads its first slice
#pragma unroll
        for (int j = 0; j < FM + FN; ++j) read1(fa0, fb0, 0, 0, j, std::bool_constant<KM>{}, std::bool_constant<KM>{});
    }
    // Step kt reads buffer kt&1.  Buffer kt&1 ^ 1 has been free since the
    // barrier of step kt-1, whose last slice started the first half of step
    // kt+1 there; the first slice of step kt adds the second half.  Before the
    // barrier of step kt this wave's loads of step kt+1 and its reads of the
    // step are complete; after it everyone's are, so buffer kt&1 takes the
    // first half of step kt+2.
    if constexpr (MODE == MODE_GRAM) {
        // Steps 0..KT-2; step KT-2 loads the first half of the last step again,
        // into a buffer nothing reads any more (keeps the loop free of branches).
        constexpr std::bool_constant<KM> km{};
        auto gram_step = [&](int kt, int buf) __attribute__((always_inline)) {
            slice(fa0, fb0, fa1, fb1, true, buf, 1, 1, (kt + 1) * kBK, buf ^ 1, LH, NL, km, km, km);
            slice(fa1, fb1, fa0, fb0, true, buf, 2, 0, 0, 0, 0, 0, km, km, km);
            slice(fa0, fb0, fa1, fb1, true, buf, 3, 0, 0, 0, 0, 0, km, km, km);
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
            asm volatile("s_barrier" ::: "memory");
            slice(fa1, fb1, fa0, fb0, true, buf ^ 1, 0, 1, min(kt + 2, KT - 1) * kBK, buf, 0, LH, km, km, km);
        };
        // Two steps per iteration, so that each step's buffer is a constant
        // and the fragment reads' addresses fold into immediate offsets.
        int kt = 0;
        for (; kt + 1 < KT - 1; kt += 2) {
            gram_step(kt, 0);
            gram_step(kt + 1, 1);
        }
        if (kt < KT - 1) gram_step(kt, 0);
    } else {
        // Steps 0..KT-3, then step KT-2 (K is a multiple of 2 kBK: buffer 0).
        // Once step KT-2 releases buffer 0, it takes the first NPRE blocks of
        // the coefficient tile while step KT-1 runs from buffer 1.
        // ma, mb: the A / B fragments of this step are read k-major.  The last
        // slice reads the next step's first slice the same way; at a switch
        // of layout the next segment reads that slice again.
        // la: the A side of step kt+2, which the last slice loads, is k-major
        // (the first slice loads the B side of step kt+1).
        auto step = [&](int kt, int buf, auto ma, auto mb, auto la) __attribute__((always_inline)) {
            slice(fa0, fb0, fa1, fb1, true, buf, 1, 1, (kt + 1) * kBK, buf ^ 1, LH, NL, ma, mb, la);
            slice(fa1, fb1, fa0, fb0, true, buf, 2, 0, 0, 0, 0, 0, ma, mb, la);
            slice(fa0, fb0, fa1, fb1, true, buf, 3, 0, 0, 0, 0, 0, ma, mb, la);
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
            asm volatile("s_barrier" ::: "memory");
            slice(fa1, fb1, fa0, fb0, true, buf ^ 1, 0, 1, (kt + 2) * kBK, buf, 0, LH, ma, mb, la);
        };
        // The last two steps: step KT-2 (buffer 0) prefetches the coefficient
        // tile into buffer 0 in its last slice while step KT-1 runs from buffer 1.
        // (The tail loads no A side: ma stands in for la.)
        auto tail = [&](auto ma, auto mb) __attribute__((always_inline)) {
            slice(fa0, fb0, fa1, fb1, true, 0, 1, 1, (KT - 1) * kBK, 1, LH, NL, ma, mb, ma);
            slice(fa1, fb1, fa0, fb0, true, 0, 2, 0, 0, 0, 0, 0, ma, mb, ma);
            slice(fa0, fb0, fa1, fb1, true, 0, 3, 0, 0, 0, 0, 0, ma, mb, ma);
            __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
            asm volatile("s_barrier" ::: "memory");
            slice(fa1, fb1, fa0, fb0, true, 1, 0, 2, 0, 0, 0, 0, ma, mb, ma);
            slice(fa0, fb0, fa1, fb1, true, 1, 1, 0, 0, 0, 0, 0, ma, mb, ma);
            slice(fa1, fb1, fa0, fb0, true, 1, 2, 0, 0, 0, 0, 0, ma, mb, ma);
            slice(fa0, fb0, fa1, fb1, true, 1, 3, 0, 0, 0, 0, 0, ma, mb, ma);
            slice(fa1, fb1, fa0, fb0, false, 0, 0, 0, 0, 0, 0, 0, ma, mb, ma);
        };
        constexpr std::false_type rm{};  // row-major fragment reads
        constexpr std::true_type kmr{};  // k-major fragment reads
        if constexpr (!LOW) {
            for (int kt = 0; kt < KT - 2; kt += 2) {  // KT - 2 is even
                step(kt, 0, rm, rm, rm);
                step(kt + 1, 1, rm, rm, rm);
            }
            tail(rm, rm);
        } else {
            // Segments [0, ksw_a): both sides row-major; [ksw_a, ksw_b): A
            // k-major (the updates: to the end); [ksw_b, KT): both k-major.
            // Each starts at an even step (buffer 0) by waiting for the reads in
            // flight and reading its first slice in its own layout (the previous
            // step's last slice read it in the old layout: discarded, and its
            // addresses stay inside the stage buffer); the first segment is at
            // least one pair long, the others may be empty.  The first
            // segment's last pair loads the A sides of steps ksw_a, ksw_a+1,
            // k-major; after it every A load is k-major.
            auto segment = [&](int k_begin, int k_end, auto ma, auto mb, auto after) __attribute__((always_inline)) {
                // Nothing may move above this wait: the registers of the reads
                // still in flight are free to the compiler from here on.
                __builtin_amdgcn_sched_barrier(0);
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                __builtin_amdgcn_sched_barrier(0);
                if constexpr (decltype(after)::value) {
                    // With both operands lower, the compiler may also reuse
                    // those registers at the previous loop's exit: an empty
                    // use after the wait keeps them live until it.
#pragma unroll
                    for (int f = 0; f < FM; ++f) asm volatile("" ::"v"(fa0[f]));
#pragma unroll
                    for (int f = 0; f < FN; ++f) asm volatile("" ::"v"(fb0[f]));
                }
#pragma unroll
                for (int j = 0; j < FM + FN; ++j) read1(fa0, fb0, 0, 0, j, ma, mb);
                if constexpr (decltype(ma)::value) {
                    for (int kt = k_begin; kt < k_end; kt += 2) {
                        step(kt, 0, ma, mb, kmr);
                        step(kt + 1, 1, ma, mb, kmr);
                    }
                } else {
                    for (int kt = k_begin; kt < k_end - 2; kt += 2) {
                        step(kt, 0, ma, mb, rm);
                        step(kt + 1, 1, ma, mb, rm);
                    }
                    step(k_end - 2, 0, ma, mb, kmr);
                    step(k_end - 1, 1, ma, mb, kmr);
                }
            };
            segment(0, ksw_a, rm, rm, std::false_type{});
            if constexpr (LOWB) {
                segment(ksw_a, ksw_b, kmr, rm, std::true_type{});
                segment(ksw_b, KT - 2, kmr, kmr, std::true_type{});
                tail(kmr, kmr);
            } else {
                segment(ksw_a, KT - 2, kmr, rm, std::false_type{});
                tail(kmr, rm);
            }
        }
    }
    if constexpr (MODE == MODE_GRAM) {  // the Gram's last step
        constexpr std::bool_constant<KM> km{};
        const int buf = (KT - 1) & 1;
        slice(fa0, fb0, fa1, fb1, true, buf, 1, 0, 0, 0, 0, 0, km, km, km);
        slice(fa1, fb1, fa0, fb0, true, buf, 2, 0, 0, 0, 0, 0, km, km, km);
        slice(fa0, fb0, fa1, fb1, true, buf, 3, 0, 0, 0, 0, 0, km, km, km);
        slice(fa1, fb1, fa0, fb0, false, 0, 0, 0, 0, 0, 0, 0, km, km, km);
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // no DMA outlives the loop

    // Epilogue, staged through LDS so that every global access is a 16-byte
    // piece of a contiguous row segment.  TT holds the tile transposed: TT row x
    // (tile column) holds the BM tile rows y in 16-byte chunks, logical chunk c
    // at physical chunk c ^ (x ^ x>>3) (mod chunks per row).  That spreads both
    // a lane's 4 rows of one column and 8 columns gathered at one row over the
    // banks (at most 2-way).
    uint16_t* const TT = smem;   // BN rows x BM bf16 (fits in the two stages)
    auto tt = [&](int x, int y) { return x * BM + ((((y >> 3) ^ x ^ (x >> 3)) & (NCH - 1)) << 3) + (y & 7); };
    const bool diag = SYM && ti == tj;
    __syncthreads();  // every wave is done with the stage buffers

    if constexpr (MODE != MODE_GRAM && MODE != MODE_APPLY) {
        // The rest of the coefficient tile (the blocks in stage buffer 1).
        constexpr int NREST = (NSB - NPRE) / 4;  // per wave
#pragma unroll
        for (int i = 0; i < NREST; ++i) src_load(NPRE + wave * NREST + i);
        __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
        __syncthreads();
    }

    // Lane holds, for fragment (a,b) and register group q, rows y..y+3 of
    // column x: one 8-byte TT cell, combined with src in place.  The 4 FN
    // cells of a fragment row are all read before any is written (to the
    // compiler a write could alias a later read, which would serialise every
    // cell behind the LDS latency).
    // With x = wn*WTN + 32b + (lane & 31) and y = wm*WTM + 32a + 8q + 4(lane >> 5),
    // y >> 3 = yc is wave-uniform and below NCH, so tt(x, y) in bytes is
    // xb2[b] + ((yc << 4) ^ xs4[b]): one xor-add per cell.
    int xb2[FN], xs4[FN];
#pragma unroll
    for (int b = 0; b < FN; ++b) {
        const int x = wn * WTN + b * 32 + (lane & 31);
        xb2[b] = (x * BM + (lane >> 5) * 4) * 2;
        xs4[b] = ((x ^ (x >> 3)) & (NCH - 1)) << 4;
    }
    auto cell = [&](int a, int b, int q) {
        const int yc = (wm * WTM + a * 32 + q * 8) >> 3;
        return reinterpret_cast<uint2*>(reinterpret_cast<char*>(TT) + (((yc << 4) ^ xs4[b]) + xb2[b]));
    };
    auto combine_row = [&](int a) {
        uint2 s2[FN][4];
        if constexpr (MODE != MODE_GRAM) {
#pragma unroll
            for (int b = 0; b < FN; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) s2[b][q] = *cell(a, b, q);
        }
#pragma unroll
        for (int b = 0; b < FN; ++b) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[a][b][q * 4 + e];
                if constexpr (MODE != MODE_GRAM) {
                    const float sv[4] = {bf16_to_f32(s2[b][q].x & 0xffffu), bf16_to_f32(s2[b][q].x >> 16),
                                         bf16_to_f32(s2[b][q].y & 0xffffu), bf16_to_f32(s2[b][q].y >> 16)};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = MODE == MODE_POLY ? __builtin_fmaf(g.alpha, v[e], g.beta * sv[e])
                                                 : __builtin_fmaf(g.beta, sv[e], v[e]);
                }
                *cell(a, b, q) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            }
        }
    };

    const MuonMatDesc& d = descs.d[bat];
    const bool tall = MODE == MODE_APPLY && d.tall;
    // Transposed orientation, from TT rows: row (tj*BN + x) of the output holds
    // TT row x.  Symmetric products: the mirror block (the tile itself on the
    // diagonal); UPDATE: X^T; APPLY: the parameter of a tall matrix.
    // k-blocked outputs: each wave writes 8 rows x 128 bytes of one panel (one
    // contiguous KB) per piece, and piece `it` covers tile rows y in
    // [64 (it / 8), +64) when BM = 256; otherwise 2 rows x 32 chunks.
    const bool has_tr = SYM || (MODE == MODE_UPDATE && g.ct) || tall;
    constexpr bool PANEL = KB && MODE != MODE_APPLY;
    constexpr int NT = BN * NCH / kGemmThreads;  // transposed pieces per thread
    auto store_tr = [&](int it) {
        const int k = it * kGemmThreads + tid;
        const int x = PANEL ? (k >> 3) % BN : k / NCH;
        const int c = PANEL ? ((k >> 3) / BN) * 8 + (k & 7) : k % NCH;
        const uint4 w = *reinterpret_cast<const uint4*>(TT + x * BM + (((c ^ x ^ (x >> 3)) & (NCH - 1)) << 3));
        const int64_t orow = int64_t(tj) * BN + x, ocol = int64_t(ti) * BM + c * 8;
        // Symmetric products: the mirror block (rows_t = mp); UPDATE: X^T (rows_t = np).
        const int64_t off = KB ? xoff(1, rows_t, 0, orow, ocol) : orow * (SYM ? g.ldc : g.ldct) + ocol;
        uint16_t* dst = SYM ? g.c + bat * g.c_bs + off : g.ct + bat * g.ct_bs + off;
        *reinterpret_cast<uint4*>(dst) = w;
    };
    // Direct orientation, gathered from TT columns: row (ti*BM + y) of the
    // output holds TT[x][y] over x.  Symmetric products: the tile's own block
    // (off the diagonal); UPDATE: X; APPLY: the parameter of a wide matrix.
    // Two transpose reads give a lane 8 consecutive columns of one row: in a
    // 16-lane group, lane j names TT[xc + j/4][yb + 4(j%4) ..], so lane i
    // receives C[yb + i][xc .. xc+3] (and xc+4 .. xc+7 from the second read).
    // A group covers 16 rows x 8 columns, the 4 groups of a wave adjacent
    // 8-column pieces of the same rows (2-way LDS bank conflicts at most);
    // piece `it` covers rows y in [16 (it / 2), +16) when BM = 256.
    const bool has_dir = (SYM && !diag) || (MODE == MODE_UPDATE && g.c) || (MODE == MODE_APPLY && !tall);
    constexpr int NXQ = BN / 32;                // 32-column pieces of a 16-row band
    constexpr int NIT = (BM / 16) * NXQ / 4;    // direct pieces per wave
    const int gi = lane & 15, grp = lane >> 4;
    auto coords = [&](int it, int64_t& orow, int64_t& ocol) {
        const int t = it * 4 + wave;
        orow = int64_t(ti) * BM + (t / NXQ) * 16 + gi;
        ocol = int64_t(tj) * BN + (t % NXQ) * 32 + grp * 8;
    };
    auto gather = [&](int it, int64_t& orow, int64_t& ocol) {
        const int t = it * 4 + wave;
        const int yb = (t / NXQ) * 16, xc = (t % NXQ) * 32 + grp * 8;
        const int xr = xc + (gi >> 2), yr = yb + 4 * (gi & 3);
        const uint2 lo = lds_read_tr16(TT + tt(xr, yr)), hi = lds_read_tr16(TT + tt(xr + 4, yr));
        coords(it, orow, ocol);
        return make_uint4(lo.x, lo.y, hi.x, hi.y);
    };
    auto store_dir = [&](int it) {
        int64_t orow, ocol;
        const uint4 wv = gather(it, orow, ocol);
        const int64_t off = KB ? xoff(1, int64_t(g.tiles_m) * BM, 0, orow, ocol)  // X, A or B k-blocked
                               : orow * g.ldc + ocol;
        *reinterpret_cast<uint4*>(g.c + bat * g.c_bs + off) = wv;
    };

    // k-blocked outputs (every product but APPLY): each store is a 16-byte
    // buffer store at a 32-bit byte offset inside one output matrix, the sum of
    // a per-lane part fixed for the tile (voffset) and a wave-uniform part per
    // piece (soffset), so no per-store address arithmetic is left; a batch's
    // LDS reads are all issued before its stores, so the batch waits on the
    // LDS latency once.  With XP = BN/32 and NXQ = BN/32:
    //   transposed piece it (x = (it%XP)*32 + tid/8, chunk c = (it/XP)*8 + tid%8):
    //     (ti*BM/64 + it/XP)*rows_t*128 + (tj*BN + (it%XP)*32)*128 + tid*16
    //   direct piece it (t = 4*it + wave):
    //     (tj*BN/64 + (t%NXQ)/2)*rows_x*128 + (ti*BM + (t/NXQ)*16)*128 + ((t%NXQ)&1)*64
    //     + (lane%16)*128 + (lane/16)*16
    // Diagonal tiles of the symmetric products take the transposed orientation
    // only: the block equals its mirror, and the MFMA result is exactly
    // symmetric (element (i,j) and (j,i) are the same products summed in the
    // same order), which the symmetry tests check bit for bit.
    if constexpr (PANEL) {
        constexpr int XP = BN / 32;
        const int64_t rows_x = int64_t(g.tiles_m) * BM;
        uint16_t* const out_tr = SYM ? g.c + bat * g.c_bs : g.ct + bat * g.ct_bs;
        uint16_t* const out_dir = g.c + bat * g.c_bs;
        const __amdgpu_buffer_rsrc_t r_tr = make_rsrc(out_tr, (SYM ? g.c_bs : g.ct_bs) * 2);
        const __amdgpu_buffer_rsrc_t r_dir = make_rsrc(out_dir, g.c_bs * 2);
        const int vo_tr = tid * 16, vo_dir = (lane & 15) * 128 + (lane >> 4) * 16;
        const int base_tr = int((int64_t(ti) * (BM / 64) * rows_t + int64_t(tj) * BN) * 128);
        const int base_dir = int((int64_t(tj) * (BN / 64) * rows_x + int64_t(ti) * BM) * 128);
        // lower: a symmetric product keeps only its lower triangle (the
        // transposed orientation of the tiles on and above the diagonal).
        const bool tr_on = has_tr, dir_on = has_dir && !(SYM && g.lower);
        auto tr_read = [&](int it) {
            const int x = (it % XP) * 32 + (tid >> 3), c = (it / XP) * 8 + (tid & 7);
            return *reinterpret_cast<const uint4*>(TT + x * BM + (((c ^ x ^ (x >> 3)) & (NCH - 1)) << 3));
        };
        auto tr_soff = [&](int it) {
            return __builtin_amdgcn_readfirstlane(base_tr + (it / XP) * int(rows_t) * 128 + (it % XP) * 4096);
        };
        auto dir_soff = [&](int it) {
            const int t = it * 4 + wave;
            return __builtin_amdgcn_readfirstlane(base_dir + ((t % NXQ) / 2) * int(rows_x) * 128 + (t / NXQ) * 2048 +
                                                  ((t % NXQ) & 1) * 64);
        };
        // Pieces it0 .. it0+NB-1 of both orientations (NB = 12 for the
        // 128 x 192 tile's 12 transposed pieces per thread: one batch).
        constexpr int NB = NT % 8 == 0 ? 8 : NT;
        typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
        auto vec = [](uint4 w) { return u32x4_t{w.x, w.y, w.z, w.w}; };
        auto store_batch = [&](int it0) {
            uint4 vt[NB], vd[NB];
            if (tr_on) {
#pragma unroll
                for (int u = 0; u < NB; ++u) vt[u] = tr_read(it0 + u);
            }
            if (dir_on) {
#pragma unroll
                for (int u = 0; u < NB; ++u) {
                    int64_t orow, ocol;
                    vd[u] = gather(it0 + u, orow, ocol);
                }
            }
            if (tr_on) {
#pragma unroll
                for (int u = 0; u < NB; ++u)
                    __builtin_amdgcn_raw_buffer_store_b128(vec(vt[u]), r_tr, vo_tr, tr_soff(it0 + u), 0);
            }
            if (dir_on) {
#pragma unroll
                for (int u = 0; u < NB; ++u)
                    __builtin_amdgcn_raw_buffer_store_b128(vec(vd[u]), r_dir, vo_dir, dir_soff(it0 + u), 0);
            }
        };
        if constexpr (BM == 256) {
            // Combine fragment rows 0-1 (tile rows y in [0, 64) and [128, 192),
            // both wave rows), store those bands (pieces 0-7 and 16-23), then
            // combine rows 2-3 while the first stores drain (pieces 8-15, 24-31).
            static_assert(FM == 4 && FN == 4 && NT == 32 && NIT == 32, "band layout of the 256 tile");
            combine_row(0);
            combine_row(1);
            __syncthreads();
            store_batch(0);
            store_batch(16);
            combine_row(2);
            combine_row(3);
            __syncthreads();
            store_batch(8);
            store_batch(24);
        } else {
            static_assert(NT == NB && (BN == 128 ? NIT == 8 : NIT == 12), "piece layout of the 128-row tiles");
#pragma unroll
            for (int a = 0; a < FM; ++a) combine_row(a);
            __syncthreads();
            store_batch(0);
        }
        return;
    }

    if constexpr (MODE == MODE_APPLY) {
        // APPLY: the parameter's own orientation, from TT rows (a tall
        // matrix: parameter row tj*BN + x holds TT row x) or gathered from TT
        // columns (a wide one), U pieces of 8 elements per thread at a time.
        // The first batch's parameter loads go out before the coefficient
        // wait and the combine, so their HBM latency passes under them: the
        // rest of the coefficient tile is issued first, and the wait lets
        // exactly those parameter loads stay in flight (apply_begin_buf
        // issues a fixed number per piece).  No fence from here on: the
        // barriers wait for LDS only (lgkmcnt), so the loads stay in flight.
        constexpr int U = NT % 8 == 0 ? 8 : 6;  // pieces per batch (NT == NIT pieces per thread)
        static_assert(NT == NIT && NT % U == 0, "whole batches");
        constexpr int NREST = (NSB - NPRE) / 4;  // per wave
        const bool bf = (d.flags & MAMW_BF16_PARAM) != 0;
        // Parameter elements the tile covers, from `base` on (rows tj*BN.. of
        // a tall matrix, ti*BM.. of a wide one); at most 2^28 of them.
        const int64_t cols = d.cols;
        const int64_t base = tall ? int64_t(tj) * BN * cols + int64_t(ti) * BM : int64_t(ti) * BM * cols + int64_t(tj) * BN;
        const int64_t span = (tall ? int64_t(BN - 1) : int64_t(BM - 1)) * cols + (tall ? BM : BN);
        const int64_t avail = max(int64_t(0), min(span, d.rows * d.cols - base));
        const int esz = bf ? 2 : 4;
        const __amdgpu_buffer_rsrc_t rp = make_rsrc(reinterpret_cast<const char*>(d.param) + base * esz, avail * esz);
        auto where = [&](int it, int64_t& orow, int64_t& ocol, int64_t& cap, int64_t& left) {
            if (tall) {
                const int k = it * kGemmThreads + tid;
                orow = int64_t(tj) * BN + k / NCH;
                ocol = int64_t(ti) * BM + (k % NCH) * 8;
                cap = orow < g.n ? 8 : 0;
                left = g.m - ocol;
            } else {
                coords(it, orow, ocol);
                cap = orow < g.m ? 8 : 0;
                left = g.n - ocol;
            }
        };
        auto value = [&](int it) {
            if (tall) {
                const int k = it * kGemmThreads + tid, x = k / NCH, c = k % NCH;
                return *reinterpret_cast<const uint4*>(TT + x * BM + (((c ^ x ^ (x >> 3)) & (NCH - 1)) << 3));
            }
            int64_t orow, ocol;
            return gather(it, orow, ocol);
        };
        // ntp: the tall path's non-temporal parameter accesses
        auto run = [&](auto ntp) __attribute__((always_inline)) {
            constexpr bool NTP = decltype(ntp)::value;
            ApplyPiece pc[U];
#pragma unroll
            for (int i = 0; i < NREST; ++i) src_load(NPRE + wave * NREST + i);
            // The parameter loads must follow the coefficient DMA in issue
            // order (the wait below counts on it): nothing moves across this.
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int u = 0; u < U; ++u) {
                int64_t orow, ocol, cap, left;
                where(u, orow, ocol, cap, left);
                apply_begin_buf<NTP>(d, pc[u], orow, ocol, cap, left, rp, base);
            }
            __builtin_amdgcn_sched_barrier(0);
            // The coefficient tile is complete once at most the U (bf16) or
            // 2U (fp32) parameter loads issued after it remain.
            if (bf)
                __builtin_amdgcn_s_waitcnt(0x0070 | (U & 15) | ((U >> 4) << 14));
            else
                __builtin_amdgcn_s_waitcnt(0x0070 | ((2 * U) & 15) | (((2 * U) >> 4) << 14));
            asm volatile("s_barrier" ::: "memory");
#pragma unroll
            for (int a = 0; a < FM; ++a) combine_row(a);
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the combined tile is in LDS
            asm volatile("s_barrier" ::: "memory");
#pragma unroll
            for (int u = 0; u < U; ++u) pc[u].w = value(u);
#pragma unroll
            for (int u = 0; u < U; ++u) apply_end<NTP>(d, pc[u], g.keep);
            for (int it0 = U; it0 < NT; it0 += U) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    int64_t orow, ocol, cap, left;
                    where(it0 + u, orow, ocol, cap, left);
                    apply_begin<NTP>(d, pc[u], orow, ocol, cap, left);
                    pc[u].w = value(it0 + u);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) apply_end<NTP>(d, pc[u], g.keep);
            }
        };
        if (tall)
            run(std::true_type{});
        else
            run(std::false_type{});
        return;
    }

#pragma unroll
    for (int a = 0; a < FM; ++a) combine_row(a);
    __syncthreads();
    if (diag) {
        // Diagonal tile of a symmetric product: the upper triangle (y <= x) is
        // authoritative; each lower element takes its mirror, so the output is
        // exactly symmetric.  Reads touch only upper cells, writes only lower.
        for (int k = tid; k < BM * NCH; k += kGemmThreads) {
            const int y = k / NCH, xc = (k % NCH) * 8;
            if (xc >= y) continue;
            const uint4 w = *reinterpret_cast<const uint4*>(TT + tt(y, xc));  // elements (xc..xc+7, y)
            const uint16_t* hv = reinterpret_cast<const uint16_t*>(&w);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (xc + j < y) TT[tt(xc + j, y)] = hv[j];
        }
        __syncthreads();
    }


    if (has_tr) {
#pragma unroll 8
        for (int it = 0; it < NT; ++it) store_tr(it);
    }
    if (has_dir) {
#pragma unroll 4
        for (int it = 0; it < NIT; ++it) store_dir(it);
    }
}

// ---------------------------------------------------------------------------
// bf16 transpose, 64 x 64 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_bf16_kernel(const uint16_t* __restrict__ src,
                                                             uint16_t* __restrict__ dst, int64_t rows,
                                                             int64_t cols, int tiles_c) {
    __shared__ uint16_t t[64][64 + 2];
    const int tid = threadIdx.x, bat = blockIdx.y;
    const int64_t r0 = int64_t(blockIdx.x / tiles_c) * 64, c0 = int64_t(blockIdx.x % tiles_c) * 64;
    const uint16_t* s = src + bat * rows * cols;
    uint16_t* o = dst + bat * rows * cols;
    for (int i = tid; i < 64 * 64; i += 256) {
        const int rl = i >> 6, cl = i & 63;
        const int64_t r = r0 + rl, c = c0 + cl;
        t[cl][rl] = (r < rows && c < cols) ? s[r * cols + c] : uint16_t(0);
    }
    __syncthreads();
    for (int i = tid; i < 64 * 64; i += 256) {
        const int cl = i >> 6, rl = i & 63;
        const int64_t r = r0 + rl, c = c0 + cl;
        if (r < rows && c < cols) o[c * rows + r] = t[cl][rl];
    }
}

// ---------------------------------------------------------------------------
// Host-side launch helpers.

// `flops` is the launch's algorithmic work: batch * (m^2 n | m^3 | 2 m^2 n) on
// the unpadded m, n for the Gram (symmetric half), polynomial and update.
// Tile codes: 128, 256 (square), kTile128x192 (the k-blocked updates with a
// lower-triangle B only).
constexpr int kTile128x192 = 192;

template <int MODE>
hipError_t launch_gemm(int tile, const GemmArgs& g, const MuonBatchDescs& d, int batch, double flops,
                       hipStream_t s) {
    // Products with an epilogue coefficient peel the last two k steps and
    // prefetch into stage buffer 0 during the last one: K is a multiple of 2 kBK.
    if (g.K < kBK || g.K % kBK != 0 || (MODE != MODE_GRAM && g.K % (2 * kBK) != 0)) return hipErrorInvalidValue;
    GemmArgs ga = g;
    ga.tiles_per_matrix = (MODE == MODE_GRAM || MODE == MODE_POLY) ? g.tiles_m * (g.tiles_m + 1) / 2
                                                                   : g.tiles_m * g.tiles_n;
    dim3 grid(unsigned(ga.tiles_per_matrix) * unsigned(batch));
    const int32_t kid = MODE == MODE_GRAM ? K_NS_GRAM : MODE == MODE_POLY ? K_NS_POLY
                      : MODE == MODE_UPDATE ? K_NS_UPDATE : K_NS_APPLY;
    const bool kb = g.xkb != 0;
    const bool km = MODE == MODE_GRAM && kb && g.kmajor;
    const bool low = MODE != MODE_GRAM && kb && g.a_low;
    // tile and the KB, KM, LOW template flags
    const int32_t variant = 8 * tile + (low ? 4 : 0) + (km ? 2 : 0) + (kb ? 1 : 0);
    const dim3 block(kGemmThreads);
    if constexpr (MODE == MODE_UPDATE || MODE == MODE_APPLY) {
        if (tile == kTile128x192) {
            if (!low) return hipErrorInvalidValue;
            return launch(kid, variant, flops, 0.0, ns_gemm_kernel<128, MODE, true, false, true, 192>, grid, block,
                          s, ga, d);
        }
    }
    if (tile == kTile128x192) return hipErrorInvalidValue;
    if constexpr (MODE != MODE_GRAM) {
        if (low) {
            if (tile == 256)
                return launch(kid, variant, flops, 0.0, ns_gemm_kernel<256, MODE, true, false, true>, grid, block, s,
                              ga, d);
            return launch(kid, variant, flops, 0.0, ns_gemm_kernel<128, MODE, true, false, true>, grid, block, s, ga,
                          d);
        }
    }
    if constexpr (MODE == MODE_GRAM) {
        if (kb && g.kmajor) {
            if (tile == 256)
                return launch(kid, variant, flops, 0.0, ns_gemm_kernel<256, MODE, true, true>, grid, block, s, ga, d);
            return launch(kid, variant, flops, 0.0, ns_gemm_kernel<128, MODE, true, true>, grid, block, s, ga, d);
        }
    }
    if (kb) {
        if (tile == 256)
            return launch(kid, variant, flops, 0.0, ns_gemm_kernel<256, MODE, true>, grid, block, s, ga, d);
        return launch(kid, variant, flops, 0.0, ns_gemm_kernel<128, MODE, true>, grid, block, s, ga, d);
    }
    if (tile == 256) return launch(kid, variant, flops, 0.0, ns_gemm_kernel<256, MODE, false>, grid, block, s, ga, d);
    return launch(kid, variant, flops, 0.0, ns_gemm_kernel<128, MODE, false>, grid, block, s, ga, d);
}

GemmArgs gram_args(const uint16_t* X, uint16_t* A, int64_t mp, int64_t kp, int tile) {
    GemmArgs g{};
    g.aop = X;
    g.bop = X;
    g.a_bs = g.b_bs = mp * kp;
    g.lda = g.ldb = kp;
    g.K = int(kp);
    g.tiles_m = g.tiles_n = int(mp / tile);
    g.c = A;
    g.c_bs = mp * mp;
    g.ldc = mp;
    g.alpha = 1.f;
    return g;
}

// A = X X^T from k-blocked XT (np x mp): both operands read k-major.
GemmArgs gram_kmajor_args(const uint16_t* XT, uint16_t* A, int64_t mp, int64_t np, int tile) {
    GemmArgs g = gram_args(XT, A, mp, np, tile);
    g.lda = g.ldb = np;  // rows of X^T: the panel height
    g.kmajor = 1;
    return g;
}

GemmArgs poly_args(const uint16_t* A, uint16_t* B, int64_t mp, int tile, float b, float c) {
    GemmArgs g{};
    g.aop = A;
    g.bop = A;
    g.a_bs = g.b_bs = mp * mp;
    g.lda = g.ldb = mp;
    g.K = int(mp);
    g.tiles_m = g.tiles_n = int(mp / tile);
    g.c = B;
    g.c_bs = mp * mp;
    g.ldc = mp;
    g.src = A;
    g.src_bs = mp * mp;
    g.lds = mp;
    g.alpha = c;
    g.beta = b;
    return g;
}

// out = a X + B X with X^T = XT as operand and epilogue source; tile_n: the
// tile's edge along n (the tile's rows of X^T).
GemmArgs update_args(const uint16_t* B, const uint16_t* XT, uint16_t* X, uint16_t* XTn, int64_t mp,
                     int64_t np, int tile, float a, int tile_n = 0) {
    GemmArgs g{};
    g.aop = B;
    g.bop = XT;
    g.a_bs = mp * mp;
    g.b_bs = np * mp;
    g.lda = mp;
    g.ldb = mp;
    g.K = int(mp);
    g.tiles_m = int(mp / tile);
    g.tiles_n = int(np / (tile_n ? tile_n : tile));
    g.c = X;
    g.c_bs = mp * np;
    g.ldc = np;
    g.ct = XTn;
    g.ct_bs = np * mp;
    g.ldct = mp;
    g.src = XT;
    g.src_bs = np * mp;
    g.lds = mp;
    g.alpha = 1.f;
    g.beta = a;
    return g;
}

}  // namespace
}  // namespace mamw

using namespace mamw;

extern "C" int mamw_muon_workspace_bytes(int batch, int64_t rows, int64_t cols, int ns_steps,
                                         size_t* bytes) {
    if (!bytes) return MAMW_ERR_NULL;
    MuonPlan p;
    int st = muon_plan(batch, rows, cols, ns_steps, &p);
    if (st != MAMW_OK) return st;
    *bytes = p.bytes;
    return MAMW_OK;
}

namespace {
int muon_step_impl(const mamw_muon_matrix* mats, int batch, double lr, double weight_decay, double beta,
                   int nesterov, float a, float b, float c, int ns_steps, float eps, void* workspace,
                   size_t workspace_bytes, const float* grad_scale, const float* found_inf,
                   mamw_stream_t stream) {
    MuonPlan p;
    MuonBatchDescs descs;
    int st = muon_validate(mats, batch, ns_steps, workspace, workspace_bytes, &p, &descs);
    if (st != MAMW_OK) return st;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    uint16_t* X = reinterpret_cast<uint16_t*>(ws + p.off_x);
    uint16_t* XT[2] = {reinterpret_cast<uint16_t*>(ws + p.off_xt0),
                       reinterpret_cast<uint16_t*>(ws + p.off_xt1)};
    uint16_t* A = reinterpret_cast<uint16_t*>(ws + p.off_a);
    uint16_t* Bm = reinterpret_cast<uint16_t*>(ws + p.off_b);
    float* part = reinterpret_cast<float*>(ws + p.off_part);
    float* inv = reinterpret_cast<float*>(ws + p.off_inv);
    // Scalars as torch forms them: lerp weights and 1 - lr*wd from double.
    const float keep = float(1.0 - lr * weight_decay);

    PrepArgs pa{};
    pa.x = X;
    pa.xt = XT[0];
    pa.part = part;
    pa.mp = p.mp;
    pa.np = p.np;
    pa.prep_tiles = p.prep_tiles;
    pa.tiles_j = int(p.np / kPrepTile);
    pa.w_mom = float(1.0 - beta);
    pa.w_nest = float(beta);
    // Workspace matrices k-blocked whenever a whole matrix's byte offsets fit the
    // 31-bit buffer offsets.
    pa.xkb = p.xkb;
    // k-blocked: the Gram reads X^T k-major, so X is needed by nothing: prep
    // writes X^T, the scale pass rescales it in place and the updates write
    // X^T only.  Row-major (matrices too large for 31-bit offsets): the Gram
    // reads X, which prep writes, the scale pass rescales and transposes, and
    // every update writes beside X^T.
    const bool kmajor = pa.xkb != 0;
    pa.xt_direct = kmajor ? 1 : 0;
    if (kmajor) pa.x = nullptr;  // no X in a k-blocked workspace
    pa.grad_scale = grad_scale;
    pa.found_inf = found_inf;
    const double B = double(batch), m = double(p.m), n = double(p.n);
    dim3 pgrid(unsigned(p.prep_tiles / 2), unsigned(batch));  // two prep units per block
    // prep: read grad, momentum; write momentum, X^T or X (4 + 4 + 4 + 2 bytes per element)
    const double prep_bytes = 14.0 * B * m * n;
    hipError_t e = nesterov ? launch(K_MUON_PREP, 1, 0.0, prep_bytes, muon_prep_kernel<true>, pgrid, dim3(256), s,
                                     descs, pa)
                            : launch(K_MUON_PREP, 0, 0.0, prep_bytes, muon_prep_kernel<false>, pgrid, dim3(256), s,
                                     descs, pa);
    if (e != hipSuccess) return int(e);
    e = launch(K_MUON_NORM, 0, 0.0, 4.0 * B * double(p.prep_tiles), muon_norm_kernel, dim3(unsigned(batch)),
               dim3(256), s, static_cast<const float*>(part), p.prep_tiles, eps, inv);
    if (e != hipSuccess) return int(e);
    // scale: read X^T, write X^T (2 + 2 bytes per padded element; mp and np are
    // multiples of 128, so 8192 elements per block divide each matrix); or
    // read X, write X and X^T (2 + 2 + 2 bytes), two prep units per block
    // Non-temporal in-place scaling once the group's X^T exceeds the 256 MiB
    // memory-side cache.
    const bool scale_nt = B * double(p.mp) * double(p.np) * 2.0 > double(256u << 20);
    if (kmajor)
        e = launch(K_MUON_SCALE, scale_nt ? 3 : 1, 0.0, 4.0 * B * double(p.mp) * double(p.np),
                   scale_nt ? muon_scale_kernel<true, true> : muon_scale_kernel<true, false>,
                   dim3(unsigned(p.mp * p.np / 8192), unsigned(batch)), dim3(256), s, pa,
                   static_cast<const float*>(inv));
    else
        e = launch(K_MUON_SCALE, 0, 0.0, 6.0 * B * double(p.mp) * double(p.np), muon_scale_kernel<false>,
                   dim3(unsigned(p.prep_tiles / 2), unsigned(batch)), dim3(256), s, pa,
                   static_cast<const float*>(inv));
    if (e != hipSuccess) return int(e);

    if (ns_steps == 0) {
        return int(launch(K_MUON_APPLY0, 0, 0.0, 10.0 * B * m * n, muon_apply0_kernel, dim3(1024, unsigned(batch)),
                          dim3(256), s, descs, pa, keep));
    }
    const double f_gram = B * m * m * n, f_poly = B * m * m * m, f_upd = 2.0 * B * m * m * n;
    // The updates take 256 x 256 tiles from m = 1024 when the padded shape
    // allows (each output element accumulates the same products in the same
    // order under either tile, so the result does not depend on it): their
    // grids hold mp/256 x np/256 tiles per matrix, enough to fill the GPU, and
    // the larger tile halves the operand traffic per flop (1024 x 4096
    // measured 11-13% faster; at m = 768 the 128 tile stays ahead).
    const int utile = (p.tile == 128 && p.m >= 1024 && p.mp % 256 == 0 && p.np % 256 == 0) ? 256 : p.tile;
    // A = X X^T and B = bA + cAA are written as their lower triangles only
    // (the symmetric products' cheaper orientation); the polynomial and the
    // updates read the blocks above the diagonal transposed.  Needs the
    // k-blocked layout, one tile size for all three products (the blocks of A
    // and B are the next products' k blocks) and at least two block rows.
    const bool lower = kmajor && utile == p.tile && p.mp >= 2 * p.tile;
    // 128 x 192 update tiles (two workgroups per CU, 17% less operand traffic
    // per flop than 128 x 128) where the class runs 128 tiles throughout, n
    // pads to a multiple of 192 and the grid holds at least 1.5 rounds of
    // 2 x 256 workgroups (GPT-2's 24 x 768 x 3072 class: update -6%, APPLY
    // -7%; 12 x 768 x 2304, 864 tiles: update -2%; smaller grids leave CUs
    // idle: 12 x 768 x 768, 288 tiles, +22%).
    const bool rect = utile == 128 && lower && p.np % 192 == 0 &&
                      int64_t(batch) * (p.mp / 128) * (p.np / 192) >= 768;
    const int ucode = rect ? kTile128x192 : utile;
    int cur = 0;
    for (int it = 0; it < ns_steps; ++it) {
        const bool last = (it == ns_steps - 1);
        GemmArgs gg = kmajor ? gram_kmajor_args(XT[cur], A, p.mp, p.np, p.tile) : gram_args(X, A, p.mp, p.np, p.tile);
        gg.xkb = pa.xkb;
        gg.lower = lower ? 1 : 0;
        e = launch_gemm<MODE_GRAM>(p.tile, gg, descs, batch, f_gram, s);
        if (e != hipSuccess) return int(e);
        GemmArgs gp = poly_args(A, Bm, p.mp, p.tile, b, c);
        gp.xkb = pa.xkb;
        gp.lower = lower ? 1 : 0;
        gp.a_low = lower ? 1 : 0;
        e = launch_gemm<MODE_POLY>(p.tile, gp, descs, batch, f_poly, s);
        if (e != hipSuccess) return int(e);
        GemmArgs gu = update_args(Bm, XT[cur], kmajor ? nullptr : X, last ? nullptr : XT[cur ^ 1], p.mp, p.np,
                                  utile, a, rect ? 192 : 0);
        gu.xkb = pa.xkb;
        gu.a_low = lower ? 1 : 0;
        if (last) {
            gu.found_inf = found_inf;
            gu.keep = keep;
            gu.m = p.m;
            gu.n = p.n;
            e = launch_gemm<MODE_APPLY>(ucode, gu, descs, batch, f_upd, s);
        } else {
            e = launch_gemm<MODE_UPDATE>(ucode, gu, descs, batch, f_upd, s);
        }
        if (e != hipSuccess) return int(e);
        cur ^= 1;
    }
    return MAMW_OK;
}
}  // namespace

extern "C" int mamw_muon_step(const mamw_muon_matrix* mats, int batch, double lr, double weight_decay,
                              double beta, int nesterov, float a, float b, float c, int ns_steps,
                              float eps, void* workspace, size_t workspace_bytes,
                              mamw_stream_t stream) {
    return muon_step_impl(mats, batch, lr, weight_decay, beta, nesterov, a, b, c, ns_steps, eps, workspace,
                          workspace_bytes, nullptr, nullptr, stream);
}

// ---------------------------------------------------------------------------
// mamw_muon_step_noalloc: the Muon workspace in a file-scope device array of
// fixed size instead of caller memory.  Each GPU the library runs on holds its
// own copy from module load until the process ends; host code reaches it only
// through the address hipGetSymbolAddress returns on that device (the array's
// name in host code is a host-side stand-in, not a device address).

static __device__ __align__(256) unsigned char scratch[MAMW_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch` per device; NULL until resolved

// Device address of `scratch` on the current device, resolved on the first
// call on that device and kept.
hipError_t scratch_address(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}
}  // namespace

extern "C" int mamw_muon_step_noalloc(const mamw_muon_matrix* mats, int batch, double lr, double weight_decay,
                                      double beta, int nesterov, float a, float b, float c, int ns_steps,
                                      float eps, mamw_stream_t stream) {
    // Host validation first, against a stand-in workspace address that no
    // caller buffer can overlap (the real array is the library's own), so
    // every rejection precedes the first HIP call.
    MuonPlan p;
    MuonBatchDescs descs;
    void* const stand_in = reinterpret_cast<void*>(uintptr_t(kWsAlign));
    int st = muon_validate(mats, batch, ns_steps, stand_in, ~size_t(0) - kWsAlign, &p, &descs);
    if (st != MAMW_OK) return st;
    if (p.bytes > size_t(MAMW_NOALLOC_SCRATCH_BYTES)) return MAMW_ERR_SCRATCH;
    void* ws = nullptr;
    const hipError_t e = scratch_address(&ws);
    if (e != hipSuccess) return int(e);
    // No per-dispatch profiler events here: creating them would allocate.
    ProfSuspend no_events;
    return muon_step_impl(mats, batch, lr, weight_decay, beta, nesterov, a, b, c, ns_steps, eps, ws,
                          size_t(MAMW_NOALLOC_SCRATCH_BYTES), nullptr, nullptr, stream);
}

extern "C" int mamw_muon_step_amp(const mamw_muon_matrix* mats, int batch, double lr, double weight_decay,
                                  double beta, int nesterov, float a, float b, float c, int ns_steps,
                                  float eps, void* workspace, size_t workspace_bytes, const float* grad_scale,
                                  const float* found_inf, mamw_stream_t stream) {
    return muon_step_impl(mats, batch, lr, weight_decay, beta, nesterov, a, b, c, ns_steps, eps, workspace,
                          workspace_bytes, grad_scale, found_inf, stream);
}

namespace {
int check_ns_dims(int batch, int64_t m, int64_t k) {
    if (batch < 1 || batch > 65535) return MAMW_ERR_COUNT;
    if (m < 128 || k < 64 || m % 128 || k % 64 || m > kMaxDim || k > kMaxDim) return MAMW_ERR_SHAPE;
    return MAMW_OK;
}
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }
size_t bf16_bytes(int batch, int64_t r, int64_t c) { return size_t(batch) * size_t(r) * size_t(c) * 2; }
}  // namespace

extern "C" int mamw_ns_gram(const uint16_t* X, uint16_t* A, int batch, int64_t m, int64_t k,
                            mamw_stream_t stream) {
    int st = check_ns_dims(batch, m, k);
    if (st != MAMW_OK) return st;
    if (!X || !A) return MAMW_ERR_NULL;
    if (!al16(X) || !al16(A)) return MAMW_ERR_ALIGN;
    if (ranges_overlap(X, bf16_bytes(batch, m, k), A, bf16_bytes(batch, m, m))) return MAMW_ERR_ALIAS;
    const int tile = (m % 256 == 0) ? choose_tile(m, k, batch) : 128;
    MuonBatchDescs d{};
    return int(launch_gemm<MODE_GRAM>(tile, gram_args(X, A, m, k, tile), d, batch,
                                      double(batch) * double(m) * double(m) * double(k),
                                      static_cast<hipStream_t>(stream)));
}

extern "C" int mamw_ns_poly(const uint16_t* A, uint16_t* B, int batch, int64_t m, float b, float c,
                            mamw_stream_t stream) {
    int st = check_ns_dims(batch, m, m);
    if (st != MAMW_OK) return st;
    if (!A || !B) return MAMW_ERR_NULL;
    if (!al16(A) || !al16(B)) return MAMW_ERR_ALIGN;
    if (ranges_overlap(A, bf16_bytes(batch, m, m), B, bf16_bytes(batch, m, m))) return MAMW_ERR_ALIAS;
    const int tile = (m % 256 == 0) ? choose_tile(m, m, batch) : 128;
    MuonBatchDescs d{};
    return int(launch_gemm<MODE_POLY>(tile, poly_args(A, B, m, tile, b, c), d, batch,
                                      double(batch) * double(m) * double(m) * double(m),
                                      static_cast<hipStream_t>(stream)));
}

extern "C" int mamw_ns_update(const uint16_t* B, const uint16_t* X, const uint16_t* XT, uint16_t* out,
                              uint16_t* out_t, int batch, int64_t m, int64_t n, float a,
                              mamw_stream_t stream) {
    int st = check_ns_dims(batch, m, n);
    if (st != MAMW_OK) return st;
    if (n % 128) return MAMW_ERR_SHAPE;
    if (!B || !X || !XT || !out) return MAMW_ERR_NULL;
    if (!al16(B) || !al16(X) || !al16(XT) || !al16(out) || (out_t && !al16(out_t))) return MAMW_ERR_ALIGN;
    // out is written from B and XT (operands and epilogue source); out_t too, and
    // from neither orientation of the other output.  out may equal X: X enters
    // only through XT.
    const size_t bb = bf16_bytes(batch, m, m), xb = bf16_bytes(batch, m, n);
    if (ranges_overlap(out, xb, B, bb) || ranges_overlap(out, xb, XT, xb)) return MAMW_ERR_ALIAS;
    if (out_t && (ranges_overlap(out_t, xb, B, bb) || ranges_overlap(out_t, xb, XT, xb) ||
                  ranges_overlap(out_t, xb, out, xb)))
        return MAMW_ERR_ALIAS;
    (void)X;  // X enters through its transpose XT (operand and epilogue source)
    const int tile = (m % 256 == 0 && n % 256 == 0) ? choose_tile(m, n, batch) : 128;
    MuonBatchDescs d{};
    return int(launch_gemm<MODE_UPDATE>(tile, update_args(B, XT, out, out_t, m, n, tile, a), d, batch,
                                        2.0 * double(batch) * double(m) * double(m) * double(n),
                                        static_cast<hipStream_t>(stream)));
}

extern "C" int mamw_transpose_bf16(const uint16_t* src, uint16_t* dst, int batch, int64_t rows,
                                   int64_t cols, mamw_stream_t stream) {
    if (batch < 1 || batch > 65535) return MAMW_ERR_COUNT;
    if (rows < 1 || cols < 1 || rows > kMaxDim || cols > kMaxDim) return MAMW_ERR_SHAPE;
    if (!src || !dst) return MAMW_ERR_NULL;
    if (ranges_overlap(src, bf16_bytes(batch, rows, cols), dst, bf16_bytes(batch, rows, cols))) return MAMW_ERR_ALIAS;
    const int tr = int((rows + 63) / 64), tc = int((cols + 63) / 64);
    return int(launch(K_TRANSPOSE, 0, 0.0, 4.0 * double(batch) * double(rows) * double(cols), transpose_bf16_kernel,
                      dim3(unsigned(tr * tc), unsigned(batch)), dim3(256), static_cast<hipStream_t>(stream), src, dst,
                      rows, cols, tc));
}
