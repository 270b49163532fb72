// AdamW update for gfx950: one single-pass kernel over every tensor of a step.
//
// Each 256-thread block owns one 1024-element chunk of one tensor and moves it
// with non-temporal 16-byte (dwordx4) loads and stores: 4 loads per thread,
// the update, 3 stores.  Small chunks keep many short-lived waves in flight
// per CU, which measured faster than fewer, longer ones.  HBM traffic is the algorithmic minimum, 28 bytes
// per element (read p, g, m, v; write p, m, v).
//
// Arithmetic follows triton_adam.py:53-59 operation by operation in IEEE fp32
// with contraction off, so results are bit-identical to an fp32 evaluation of
// that formula (IEEE division and square root).
#include "mamw_device.h"
#include "mamw_launch.h"

#pragma clang fp contract(off)

namespace mamw {
namespace {

struct AdamWConsts {
    float lr, bias1, bias2, beta1, beta2, eps;
    float omb1, omb2, decay;  // 1-beta1, 1-beta2, 1-lr*weight_decay (fp32, as the reference)
    // Gradient-scaler step (all NULL otherwise): gradients are divided by
    // *grad_scale; a non-zero *found_inf skips the update; the bias
    // corrections are read from bias[0..1], written just before by
    // adamw_bias_kernel from the device step counter.
    const float* grad_scale;
    const float* found_inf;
    const float* bias;
    float gs;     // *grad_scale, read by the kernel
    int scaled;   // grad_scale != NULL
};

__host__ AdamWConsts make_consts(const AdamWScalars& s) {
    AdamWConsts c;
    c.lr = s.lr;
    c.bias1 = s.bias1;
    c.bias2 = s.bias2;
    c.beta1 = s.beta1;
    c.beta2 = s.beta2;
    c.eps = s.eps;
    c.omb1 = 1.0f - s.beta1;
    c.omb2 = 1.0f - s.beta2;
    c.decay = 1.0f - s.lr * s.weight_decay;
    c.grad_scale = c.found_inf = c.bias = nullptr;
    c.gs = 1.0f;
    c.scaled = 0;
    return c;
}

// Per-block set-up of a gradient-scaler step: false when the step is skipped.
__device__ __forceinline__ bool adamw_prepare(AdamWConsts& c) {
    if (c.found_inf && *c.found_inf != 0.0f) return false;
    if (c.bias) {
        c.bias1 = c.bias[0];
        c.bias2 = c.bias[1];
    }
    if (c.grad_scale) {
        c.gs = *c.grad_scale;
        c.scaled = 1;
    }
    return true;
}

__device__ __forceinline__ float4 unscale4(float4 g, const AdamWConsts& c) {
    return c.scaled ? make_float4(g.x / c.gs, g.y / c.gs, g.z / c.gs, g.w / c.gs) : g;
}

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v,
                                           const AdamWConsts& c) {
    const float mt = c.beta1 * m + c.omb1 * g;
    const float vt = c.beta2 * v + c.omb2 * (g * g);
    const float mc = mt / c.bias1;
    const float vc = vt / c.bias2;
    const float pd = c.decay * p;
    p = pd - c.lr * (mc / (sqrtf(vc) + c.eps));
    m = mt;
    v = vt;
}

// Streaming 16-byte accesses: every byte is touched once, so the loads and
// stores are non-temporal (measured: +6-8 points of HBM bandwidth over plain
// accesses on this kernel; either half alone gains nothing).
typedef float nt_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 nt_load(const float4* q) {
    const nt_f4 v = __builtin_nontemporal_load(reinterpret_cast<const nt_f4*>(q));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void nt_store(float4* q, float4 x) {
    const nt_f4 v = {x.x, x.y, x.z, x.w};
    __builtin_nontemporal_store(v, reinterpret_cast<nt_f4*>(q));
}

__device__ __forceinline__ void adamw_vec(float4& p, float4 g, float4& m, float4& v,
                                          const AdamWConsts& c) {
    adamw_elem(p.x, g.x, m.x, v.x, c);
    adamw_elem(p.y, g.y, m.y, v.y, c);
    adamw_elem(p.z, g.z, m.z, v.z, c);
    adamw_elem(p.w, g.w, m.w, v.w, c);
}

// 4-element groups of a parameter or gradient buffer: fp32 (16 bytes) or bf16
// (8 bytes, widened exactly; stores round to nearest-even).
template <bool BF16>
__device__ __forceinline__ float4 ld4(const void* base, int64_t i) {
    if constexpr (BF16) {
        typedef unsigned int nt_u2 __attribute__((ext_vector_type(2)));
        const nt_u2 w = __builtin_nontemporal_load(reinterpret_cast<const nt_u2*>(base) + i);
        return make_float4(bf16_to_f32(w.x & 0xffffu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xffffu),
                           bf16_to_f32(w.y >> 16));
    } else {
        return nt_load(reinterpret_cast<const float4*>(base) + i);
    }
}
template <bool BF16>
__device__ __forceinline__ void st4(void* base, int64_t i, float4 x) {
    if constexpr (BF16) {
        typedef unsigned int nt_u2 __attribute__((ext_vector_type(2)));
        const nt_u2 w = {pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w)};
        __builtin_nontemporal_store(w, reinterpret_cast<nt_u2*>(base) + i);
    } else {
        nt_store(reinterpret_cast<float4*>(base) + i, x);
    }
}
template <bool BF16>
__device__ __forceinline__ float ld1(const void* base, int64_t i) {
    if constexpr (BF16)
        return bf16_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
    else
        return reinterpret_cast<const float*>(base)[i];
}
template <bool BF16>
__device__ __forceinline__ void st1(void* base, int64_t i, float x) {
    if constexpr (BF16)
        reinterpret_cast<uint16_t*>(base)[i] = uint16_t(f32_to_bf16(x));
    else
        reinterpret_cast<float*>(base)[i] = x;
}

// Update elements [start, start + len) of tensor r (len <= kAdamWChunk); PB /
// GB: the parameter / gradient hold bf16.  The arithmetic is the fp32 one in
// every case.
template <bool PB, bool GB>
__device__ __forceinline__ void adamw_chunk(const AdamWRec& r, int64_t start, int len,
                                            const AdamWConsts& c) {
    const int tid = threadIdx.x;
    float* __restrict__ M = r.m + start;
    float* __restrict__ V = r.v + start;
    float4* M4 = reinterpret_cast<float4*>(M);
    float4* V4 = reinterpret_cast<float4*>(V);
    // Vector index i covers elements start + 4i .. +3 (start is a multiple of 4).
    const int64_t q0 = start >> 2;
    if (r.vec_ok && len == kAdamWChunk) {
        float4 p[kAdamWUnroll], g[kAdamWUnroll], m[kAdamWUnroll], v[kAdamWUnroll];
#pragma unroll
        for (int u = 0; u < kAdamWUnroll; ++u) {
            const int i = u * kAdamWThreads + tid;
            p[u] = ld4<PB>(r.p, q0 + i);
            g[u] = unscale4(ld4<GB>(r.g, q0 + i), c);
            m[u] = nt_load(M4 + i);
            v[u] = nt_load(V4 + i);
        }
#pragma unroll
        for (int u = 0; u < kAdamWUnroll; ++u) {
            const int i = u * kAdamWThreads + tid;
            adamw_vec(p[u], g[u], m[u], v[u], c);
            st4<PB>(r.p, q0 + i, p[u]);
            nt_store(M4 + i, m[u]);
            nt_store(V4 + i, v[u]);
        }
        return;
    }
    int scalar_from = 0;
    if (r.vec_ok) {
        const int nv = len >> 2;
        for (int i = tid; i < nv; i += kAdamWThreads) {
            float4 p = ld4<PB>(r.p, q0 + i), m = nt_load(M4 + i), v = nt_load(V4 + i);
            adamw_vec(p, unscale4(ld4<GB>(r.g, q0 + i), c), m, v, c);
            st4<PB>(r.p, q0 + i, p);
            nt_store(M4 + i, m);
            nt_store(V4 + i, v);
        }
        scalar_from = nv << 2;
    }
    for (int e = scalar_from + tid; e < len; e += kAdamWThreads) {
        float p = ld1<PB>(r.p, start + e), m = M[e], v = V[e];
        const float ge = ld1<GB>(r.g, start + e);
        adamw_elem(p, c.scaled ? ge / c.gs : ge, m, v, c);
        st1<PB>(r.p, start + e, p);
        M[e] = m;
        V[e] = v;
    }
}

// The block's chunk, dispatched on the tensor's element types (uniform per block).
__device__ __forceinline__ void adamw_chunk_any(const AdamWRec& r, int64_t start, int len,
                                                const AdamWConsts& c) {
    switch (r.flags & (MAMW_BF16_PARAM | MAMW_BF16_GRAD)) {
        case 0: adamw_chunk<false, false>(r, start, len, c); break;
        case MAMW_BF16_PARAM: adamw_chunk<true, false>(r, start, len, c); break;
        case MAMW_BF16_GRAD: adamw_chunk<false, true>(r, start, len, c); break;
        default: adamw_chunk<true, true>(r, start, len, c); break;
    }
}

__global__ __launch_bounds__(kAdamWThreads) void adamw_mt_kernel(const AdamWRec* __restrict__ recs,
                                                                  int n, AdamWConsts c) {
    if (!adamw_prepare(c)) return;
    const int64_t b = blockIdx.x;
    // Largest t with recs[t].block_begin <= b (block_begin is non-decreasing):
    // binary search with scalar loads down to a range of at most 64 records,
    // then one vector load of the range, one record per lane, and a ballot.
    // (The last level as a vector load measured +5% on the 256-tensor config-2
    // set over a binary search to the end; a 16-way scalar search gained
    // nothing.)
    int lo = 0, hi = n - 1;
    while (hi - lo >= 64) {
        const int mid = (lo + hi + 1) >> 1;
        if (recs[mid].block_begin <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    {
        const int idx = lo + int(threadIdx.x & 63);
        const bool le = idx <= hi && recs[idx].block_begin <= b;
        lo = __builtin_amdgcn_readfirstlane(lo + int(__popcll(__ballot(le))) - 1);
    }
    const AdamWRec r = recs[lo];
    const int64_t start = (b - r.block_begin) * kAdamWChunk;
    const int64_t rem = r.numel - start;
    adamw_chunk_any(r, start, rem < kAdamWChunk ? int(rem) : int(kAdamWChunk), c);
}

__global__ __launch_bounds__(kAdamWThreads) void adamw_one_kernel(AdamWRec r, AdamWConsts c) {
    if (!adamw_prepare(c)) return;
    const int64_t start = int64_t(blockIdx.x) * kAdamWChunk;
    const int64_t rem = r.numel - start;
    adamw_chunk_any(r, start, rem < kAdamWChunk ? int(rem) : int(kAdamWChunk), c);
}

}  // namespace
}  // namespace mamw

using namespace mamw;

extern "C" int mamw_adamw_tensor_step(float* param, const float* grad, float* exp_avg,
                                      float* exp_avg_sq, int64_t numel, float lr, float bias1,
                                      float bias2, float beta1, float beta2, float weight_decay,
                                      float eps, mamw_stream_t stream) {
    mamw_adamw_tensor t{param, grad, exp_avg, exp_avg_sq, numel};
    int64_t blocks = 0;
    AdamWRec r[2];  // a packed table of one tensor (the trailing record is unused here)
    int st = adamw_table_pack(&t, 1, r, sizeof(r), &blocks);
    if (st != MAMW_OK) return st;
    if (blocks == 0) return MAMW_OK;
    AdamWScalars s{lr, bias1, bias2, beta1, beta2, weight_decay, eps};
    return int(launch(K_ADAMW_ONE, 0, 0.0, 28.0 * double(numel), adamw_one_kernel, dim3(unsigned(blocks)),
                      dim3(kAdamWThreads), static_cast<hipStream_t>(stream), r[0], make_consts(s)));
}

extern "C" int mamw_adamw_table_bytes(int n_tensors, size_t* bytes) {
    return adamw_table_bytes(n_tensors, bytes);
}

extern "C" int mamw_adamw_table_pack(const mamw_adamw_tensor* tensors, int n_tensors,
                                     void* host_table, size_t table_bytes, int64_t* n_blocks) {
    return adamw_table_pack(tensors, n_tensors, host_table, table_bytes, n_blocks);
}

extern "C" int mamw_adamw_table_pack_ex(const mamw_adamw_tensor_ex* tensors, int n_tensors,
                                        void* host_table, size_t table_bytes, int64_t* n_blocks) {
    return adamw_table_pack_ex(tensors, n_tensors, host_table, table_bytes, n_blocks);
}

namespace {
// The bias corrections of a device-counter step, once per launch (rather than
// in every wave of the update): 1 - beta^step in double from the double
// betas, rounded to fp32, as the host forms them from its own counter.
__global__ __launch_bounds__(64) void adamw_bias_kernel(const float* __restrict__ step, double beta1,
                                                        double beta2, float* __restrict__ bias) {
    if (threadIdx.x == 0) {
        const double st = double(*step);
        bias[0] = float(1.0 - pow(beta1, st));
        bias[1] = float(1.0 - pow(beta2, st));
    }
}

// Host validation shared by both multi-tensor entry points, complete before
// any HIP call: MAMW_OK with *launch = false when there is nothing to do.
int adamw_mt_validate(const void* device_table, int n_tensors, int64_t n_blocks, bool* launch) {
    *launch = false;
    if (n_tensors < 0 || n_tensors > kMaxTensors) return MAMW_ERR_COUNT;
    if (n_blocks < 0 || n_blocks > int64_t(0x7fffffff)) return MAMW_ERR_NUMEL;
    if (n_blocks == 0) return MAMW_OK;
    if (n_tensors == 0) return MAMW_ERR_COUNT;
    if (!device_table) return MAMW_ERR_NULL;
    if (reinterpret_cast<uintptr_t>(device_table) % 16) return MAMW_ERR_ALIGN;
    *launch = true;
    return MAMW_OK;
}

int adamw_mt_launch(const void* device_table, int n_tensors, int64_t n_blocks, const AdamWConsts& c,
                    mamw_stream_t stream) {
    // Algorithmic bytes (28 per element) are not known here: the table is in device memory.
    return int(launch(K_ADAMW_MT, 0, 0.0, 0.0, adamw_mt_kernel, dim3(unsigned(n_blocks)), dim3(kAdamWThreads),
                      static_cast<hipStream_t>(stream), static_cast<const AdamWRec*>(device_table), n_tensors, c));
}
}  // namespace

extern "C" int mamw_adamw_mt_step(const void* device_table, int n_tensors, int64_t n_blocks,
                                  float lr, float bias1, float bias2, float beta1, float beta2,
                                  float weight_decay, float eps, mamw_stream_t stream) {
    bool go = false;
    const int st = adamw_mt_validate(device_table, n_tensors, n_blocks, &go);
    if (st != MAMW_OK || !go) return st;
    AdamWScalars s{lr, bias1, bias2, beta1, beta2, weight_decay, eps};
    return adamw_mt_launch(device_table, n_tensors, n_blocks, make_consts(s), stream);
}

extern "C" int mamw_adamw_mt_step_amp(void* device_table, int n_tensors, int64_t n_blocks,
                                      float lr, double beta1, double beta2, float weight_decay, float eps,
                                      const float* step, const float* grad_scale, const float* found_inf,
                                      mamw_stream_t stream) {
    if (!step) return MAMW_ERR_NULL;
    bool go = false;
    const int vs = adamw_mt_validate(device_table, n_tensors, n_blocks, &go);
    if (vs != MAMW_OK || !go) return vs;
    AdamWScalars s{lr, 1.0f, 1.0f, float(beta1), float(beta2), weight_decay, eps};
    AdamWConsts c = make_consts(s);
    // The table's trailing record (after n_tensors records) holds the two corrections.
    float* bias = reinterpret_cast<float*>(static_cast<AdamWRec*>(device_table) + n_tensors);
    c.bias = bias;
    c.grad_scale = grad_scale;
    c.found_inf = found_inf;
    const int st = int(launch(K_ADAMW_BIAS, 0, 0.0, 0.0, adamw_bias_kernel, dim3(1), dim3(64),
                              static_cast<hipStream_t>(stream), step, beta1, beta2, bias));
    if (st != 0) return st;
    return adamw_mt_launch(device_table, n_tensors, n_blocks, c, stream);
}
