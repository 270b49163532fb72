// Host-side planning and validation (no HIP calls).
#include "mamw_plan.h"

#include <string.h>

#include <algorithm>
#include <vector>

namespace mamw {

namespace {

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

bool overlap(const void* a, size_t na, const void* b, size_t nb) { return ranges_overlap(a, na, b, nb); }

// Across the tensors of one table (one launch runs them all at once): memory
// a tensor writes (param, exp_avg, exp_avg_sq) must not overlap memory any
// tensor reads or writes; gradients may be shared.  One sort of the byte
// ranges and a sweep, so large tables stay cheap.
struct Span {
    uintptr_t lo, hi;
    bool write;
};

int adamw_cross_alias(const mamw_adamw_tensor_ex* t, int n) {
    if (n < 2) return MAMW_OK;
    std::vector<Span> s;
    try {  // no C++ exception may cross the C ABI
        s.reserve(size_t(n) * 4);
    } catch (...) {
        return MAMW_ERR_COUNT;
    }
    for (int i = 0; i < n; ++i) {
        if (t[i].numel <= 0) continue;
        const size_t ne = size_t(t[i].numel);
        const size_t ep = (t[i].flags & MAMW_BF16_PARAM) ? 2 : 4, eg = (t[i].flags & MAMW_BF16_GRAD) ? 2 : 4;
        const void* ptr[4] = {t[i].param, t[i].exp_avg, t[i].exp_avg_sq, t[i].grad};
        const size_t len[4] = {ne * ep, ne * 4, ne * 4, ne * eg};
        for (int k = 0; k < 4; ++k) {
            const uintptr_t lo = reinterpret_cast<uintptr_t>(ptr[k]);
            s.push_back({lo, lo + len[k], k < 3});
        }
    }
    std::sort(s.begin(), s.end(), [](const Span& x, const Span& y) { return x.lo < y.lo; });
    uintptr_t end_any = 0, end_write = 0;  // furthest end of the ranges before, of any kind / written
    for (const Span& x : s) {
        if (x.lo < (x.write ? end_any : end_write)) return MAMW_ERR_ALIAS;
        end_any = std::max(end_any, x.hi);
        if (x.write) end_write = std::max(end_write, x.hi);
    }
    return MAMW_OK;
}

}  // namespace

bool ranges_overlap(const void* a, size_t na, const void* b, size_t nb) {
    uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return na && nb && pa < pb + nb && pb < pa + na;
}

// ---------------------------------------------------------------------------
// AdamW

int adamw_validate_tensor(const mamw_adamw_tensor_ex& t) {
    if (t.flags & ~(MAMW_BF16_PARAM | MAMW_BF16_GRAD) || t.reserved != 0) return MAMW_ERR_HYPER;
    if (t.numel < 0 || t.numel > kMaxNumel) return MAMW_ERR_NUMEL;
    if (t.numel == 0) return MAMW_OK;
    if (!t.param || !t.grad || !t.exp_avg || !t.exp_avg_sq) return MAMW_ERR_NULL;
    const size_t ep = (t.flags & MAMW_BF16_PARAM) ? 2 : 4, eg = (t.flags & MAMW_BF16_GRAD) ? 2 : 4;
    if (!aligned(t.param, ep) || !aligned(t.grad, eg) || !aligned(t.exp_avg, 4) || !aligned(t.exp_avg_sq, 4))
        return MAMW_ERR_ALIGN;
    // param, exp_avg, exp_avg_sq are written: they must not overlap each other
    // or the gradient.
    const size_t n = size_t(t.numel);
    const void* w[3] = {t.param, t.exp_avg, t.exp_avg_sq};
    const size_t wb[3] = {n * ep, n * 4, n * 4};
    for (int i = 0; i < 3; ++i) {
        if (overlap(w[i], wb[i], t.grad, n * eg)) return MAMW_ERR_ALIAS;
        for (int j = i + 1; j < 3; ++j)
            if (overlap(w[i], wb[i], w[j], wb[j])) return MAMW_ERR_ALIAS;
    }
    return MAMW_OK;
}

int adamw_table_bytes(int n_tensors, size_t* bytes) {
    if (!bytes) return MAMW_ERR_NULL;
    if (n_tensors < 0 || n_tensors > kMaxTensors) return MAMW_ERR_COUNT;
    *bytes = size_t(n_tensors + 1) * sizeof(AdamWRec);  // + the record the device-counter step writes
    return MAMW_OK;
}

int adamw_table_pack_ex(const mamw_adamw_tensor_ex* tensors, int n_tensors, void* host_table,
                        size_t table_bytes, int64_t* n_blocks) {
    if (!n_blocks) return MAMW_ERR_NULL;
    if (n_tensors < 0 || n_tensors > kMaxTensors) return MAMW_ERR_COUNT;
    if (n_tensors > 0 && (!tensors || !host_table)) return MAMW_ERR_NULL;
    if (n_tensors > 0 && table_bytes < size_t(n_tensors + 1) * sizeof(AdamWRec)) return MAMW_ERR_TABLE;
    AdamWRec* rec = static_cast<AdamWRec*>(host_table);
    int64_t blocks = 0;
    for (int i = 0; i < n_tensors; ++i) {
        const mamw_adamw_tensor_ex& t = tensors[i];
        int st = adamw_validate_tensor(t);
        if (st != MAMW_OK) return st;
        AdamWRec r;
        memset(&r, 0, sizeof(r));
        r.p = t.param;
        r.g = t.grad;
        r.m = t.exp_avg;
        r.v = t.exp_avg_sq;
        r.numel = t.numel;
        r.block_begin = blocks;
        r.flags = t.flags;
        // 4 elements per vector access: 16 bytes of fp32, 8 of bf16.
        r.vec_ok = aligned(t.param, (t.flags & MAMW_BF16_PARAM) ? 8 : 16) &&
                   aligned(t.grad, (t.flags & MAMW_BF16_GRAD) ? 8 : 16) && aligned(t.exp_avg, 16) &&
                   aligned(t.exp_avg_sq, 16);
        memcpy(&rec[i], &r, sizeof(r));
        blocks += (t.numel + kAdamWChunk - 1) / kAdamWChunk;
        if (blocks > int64_t(0x7fffffff)) return MAMW_ERR_NUMEL;  // grid.x limit
    }
    const int st = adamw_cross_alias(tensors, n_tensors);
    if (st != MAMW_OK) return st;
    if (n_tensors > 0) memset(&rec[n_tensors], 0, sizeof(AdamWRec));  // written by the device-counter step
    *n_blocks = blocks;
    return MAMW_OK;
}

int adamw_table_pack(const mamw_adamw_tensor* tensors, int n_tensors, void* host_table, size_t table_bytes,
                     int64_t* n_blocks) {
    if (!n_blocks) return MAMW_ERR_NULL;
    if (n_tensors < 0 || n_tensors > kMaxTensors) return MAMW_ERR_COUNT;
    if (n_tensors > 0 && (!tensors || !host_table)) return MAMW_ERR_NULL;
    if (n_tensors > 0 && table_bytes < size_t(n_tensors + 1) * sizeof(AdamWRec)) return MAMW_ERR_TABLE;
    // fp32 entries are packed one at a time through the general path; the
    // cross-tensor check then sees them together (one host array).
    AdamWRec* rec = static_cast<AdamWRec*>(host_table);
    int64_t blocks = 0;
    for (int i = 0; i < n_tensors; ++i) {
        const mamw_adamw_tensor& t = tensors[i];
        const mamw_adamw_tensor_ex e{t.param, t.grad, t.exp_avg, t.exp_avg_sq, t.numel, 0, 0};
        int64_t nb = 0;
        int st = adamw_table_pack_ex(&e, 1, &rec[i], table_bytes - size_t(i) * sizeof(AdamWRec), &nb);
        if (st != MAMW_OK) return st;
        rec[i].block_begin = blocks;
        blocks += nb;
        if (blocks > int64_t(0x7fffffff)) return MAMW_ERR_NUMEL;
    }
    if (n_tensors > 1) {
        std::vector<mamw_adamw_tensor_ex> ex;
        try {  // no C++ exception may cross the C ABI
            ex.resize(static_cast<size_t>(n_tensors));
        } catch (...) {
            return MAMW_ERR_COUNT;
        }
        for (int i = 0; i < n_tensors; ++i) {
            const mamw_adamw_tensor& t = tensors[i];
            ex[size_t(i)] = mamw_adamw_tensor_ex{t.param, t.grad, t.exp_avg, t.exp_avg_sq, t.numel, 0, 0};
        }
        const int st = adamw_cross_alias(ex.data(), n_tensors);
        if (st != MAMW_OK) return st;
    }
    *n_blocks = blocks;
    return MAMW_OK;
}

// ---------------------------------------------------------------------------
// Muon

int choose_tile(int64_t m, int64_t n, int batch) {
    // 256 x 256 tiles halve the operand traffic per flop but need enough
    // tiles to fill 256 CUs at one workgroup each.  From m = 2048 a matrix has
    // 36 or more symmetric 256-tiles.  From m = 1024 a batch of 8 or more
    // matrices has 80 or more (10 per matrix) and takes 256 tiles too, when
    // their padding adds at most 1/16 to the 128 tile's (the 1024 x 4096
    // groups of Llama-8B: class step 6.17 -> 5.76 ms with groups of 24, 24,
    // 16); smaller batches keep the 128 tile's workgroups in flight.
    if (m >= 2048) return 256;
    if (m >= 1024 && batch >= 8 &&
        round_up(m, 256) * round_up(n, 256) * 16 <= round_up(m, 128) * round_up(n, 128) * 17)
        return 256;
    return 128;
}

int muon_plan(int batch, int64_t rows, int64_t cols, int ns_steps, MuonPlan* plan) {
    if (!plan) return MAMW_ERR_NULL;
    if (batch < 1 || batch > MAMW_MUON_MAX_BATCH) return MAMW_ERR_COUNT;
    if (rows < 1 || cols < 1 || rows > kMaxDim || cols > kMaxDim) return MAMW_ERR_SHAPE;
    if (ns_steps < 0 || ns_steps >= 100) return MAMW_ERR_HYPER;
    MuonPlan p;
    memset(&p, 0, sizeof(p));
    p.batch = batch;
    p.m = rows < cols ? rows : cols;
    p.n = rows < cols ? cols : rows;
    p.tile = choose_tile(p.m, p.n, batch);
    p.mp = round_up(p.m, p.tile);
    p.np = round_up(p.n, p.tile);
    if (p.mp * p.np > kMaxMatElems) return MAMW_ERR_SHAPE;
    p.prep_tiles = (p.mp / kPrepTile) * (p.np / kPrepTile);
    p.xkb = (p.mp * p.np * 2 < (int64_t(1) << 31)) ? 1 : 0;
    const size_t B = size_t(batch);
    const size_t xe = size_t(p.mp) * size_t(p.np);  // elements of X / XT
    const size_t ae = size_t(p.mp) * size_t(p.mp);  // elements of A / B
    size_t off = 0;
    p.off_x = off;
    if (!p.xkb) off = align_ws(off + B * xe * 2);
    p.off_xt0 = off;
    off = align_ws(off + B * xe * 2);
    p.off_xt1 = off;
    if (ns_steps >= 2) off = align_ws(off + B * xe * 2);
    p.off_a = off;
    if (ns_steps >= 1) off = align_ws(off + B * ae * 2);
    p.off_b = off;
    if (ns_steps >= 1) off = align_ws(off + B * ae * 2);
    p.off_part = off;
    off = align_ws(off + B * size_t(p.prep_tiles) * 4);
    p.off_inv = off;
    off = align_ws(off + B * 4);
    p.bytes = off;
    *plan = p;
    return MAMW_OK;
}

int muon_validate(const mamw_muon_matrix* mats, int batch, int ns_steps, const void* workspace,
                  size_t workspace_bytes, MuonPlan* plan, MuonBatchDescs* descs) {
    if (!mats || !plan || !descs) return MAMW_ERR_NULL;
    if (batch < 1 || batch > MAMW_MUON_MAX_BATCH) return MAMW_ERR_COUNT;
    int st = muon_plan(batch, mats[0].rows, mats[0].cols, ns_steps, plan);
    if (st != MAMW_OK) return st;
    if (!workspace) return MAMW_ERR_WORKSPACE;
    if (!aligned(workspace, kWsAlign) || workspace_bytes < plan->bytes) return MAMW_ERR_WORKSPACE;
    memset(descs, 0, sizeof(*descs));
    for (int i = 0; i < batch; ++i) {
        const mamw_muon_matrix& M = mats[i];
        if (M.flags & ~(MAMW_BF16_PARAM | MAMW_BF16_GRAD)) return MAMW_ERR_HYPER;
        if (M.rows < 1 || M.cols < 1) return MAMW_ERR_SHAPE;
        const int64_t mi = M.rows < M.cols ? M.rows : M.cols;
        const int64_t ni = M.rows < M.cols ? M.cols : M.rows;
        if (mi != plan->m || ni != plan->n) return MAMW_ERR_SHAPE;
        if (!M.param || !M.grad || !M.momentum) return MAMW_ERR_NULL;
        const size_t ep = (M.flags & MAMW_BF16_PARAM) ? 2 : 4, eg = (M.flags & MAMW_BF16_GRAD) ? 2 : 4;
        if (!aligned(M.param, ep) || !aligned(M.grad, eg) || !aligned(M.momentum, 4)) return MAMW_ERR_ALIGN;
        const size_t ne = size_t(M.rows) * size_t(M.cols);
        const size_t nb = ne * 4, np_ = ne * ep, ng = ne * eg;
        if (overlap(M.param, np_, M.grad, ng) || overlap(M.param, np_, M.momentum, nb) ||
            overlap(M.momentum, nb, M.grad, ng))
            return MAMW_ERR_ALIAS;
        if (overlap(M.param, np_, workspace, plan->bytes) || overlap(M.momentum, nb, workspace, plan->bytes) ||
            overlap(M.grad, ng, workspace, plan->bytes))
            return MAMW_ERR_ALIAS;
        if (M.update) {
            if (!aligned(M.update, 4)) return MAMW_ERR_ALIGN;
            if (overlap(M.update, nb, M.param, np_) || overlap(M.update, nb, M.grad, ng) ||
                overlap(M.update, nb, M.momentum, nb) || overlap(M.update, nb, workspace, plan->bytes))
                return MAMW_ERR_ALIAS;
        }
        // Across entries: memory one entry writes (parameter, momentum,
        // update) must not overlap anything another entry reads or writes
        // (the batch's kernels run over all entries at once).
        const void* wi[3] = {M.param, M.momentum, M.update};
        const size_t wbi[3] = {np_, nb, M.update ? nb : 0};
        for (int j = 0; j < i; ++j) {
            const mamw_muon_matrix& N = mats[j];
            const size_t nej = size_t(N.rows) * size_t(N.cols);
            const void* wj[3] = {N.param, N.momentum, N.update};
            const size_t wbj[3] = {nej * ((N.flags & MAMW_BF16_PARAM) ? 2 : 4), nej * 4, N.update ? nej * 4 : 0};
            const size_t ngj = nej * ((N.flags & MAMW_BF16_GRAD) ? 2 : 4);
            for (int x = 0; x < 3; ++x) {
                if (overlap(wi[x], wbi[x], N.grad, ngj) || overlap(wj[x], wbj[x], M.grad, ng)) return MAMW_ERR_ALIAS;
                for (int y = 0; y < 3; ++y)
                    if (overlap(wi[x], wbi[x], wj[y], wbj[y])) return MAMW_ERR_ALIAS;
            }
        }
        MuonMatDesc& d = descs->d[i];
        d.param = M.param;
        d.grad = M.grad;
        d.mom = M.momentum;
        d.upd = M.update;
        d.rows = M.rows;
        d.cols = M.cols;
        d.slr = M.scaled_lr;
        d.tall = M.rows > M.cols ? 1 : 0;
        d.flags = M.flags;
    }
    return MAMW_OK;
}

}  // namespace mamw
