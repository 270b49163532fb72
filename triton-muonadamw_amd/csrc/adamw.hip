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
    return c;
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

// Update elements [start, start + len) of tensor r (len <= kAdamWChunk).
__device__ __forceinline__ void adamw_chunk(const AdamWRec& r, int64_t start, int len,
                                            const AdamWConsts& c) {
    const int tid = threadIdx.x;
    float* __restrict__ P = r.p + start;
    const float* __restrict__ G = r.g + start;
    float* __restrict__ M = r.m + start;
    float* __restrict__ V = r.v + start;
    if (r.vec_ok && len == kAdamWChunk) {
        float4* P4 = reinterpret_cast<float4*>(P);
        const float4* G4 = reinterpret_cast<const float4*>(G);
        float4* M4 = reinterpret_cast<float4*>(M);
        float4* V4 = reinterpret_cast<float4*>(V);
        float4 p[kAdamWUnroll], g[kAdamWUnroll], m[kAdamWUnroll], v[kAdamWUnroll];
#pragma unroll
        for (int u = 0; u < kAdamWUnroll; ++u) {
            const int i = u * kAdamWThreads + tid;
            p[u] = nt_load(P4 + i);
            g[u] = nt_load(G4 + i);
            m[u] = nt_load(M4 + i);
            v[u] = nt_load(V4 + i);
        }
#pragma unroll
        for (int u = 0; u < kAdamWUnroll; ++u) {
            const int i = u * kAdamWThreads + tid;
            adamw_vec(p[u], g[u], m[u], v[u], c);
            nt_store(P4 + i, p[u]);
            nt_store(M4 + i, m[u]);
            nt_store(V4 + i, v[u]);
        }
        return;
    }
    int scalar_from = 0;
    if (r.vec_ok) {
        const int nv = len >> 2;
        float4* P4 = reinterpret_cast<float4*>(P);
        const float4* G4 = reinterpret_cast<const float4*>(G);
        float4* M4 = reinterpret_cast<float4*>(M);
        float4* V4 = reinterpret_cast<float4*>(V);
        for (int i = tid; i < nv; i += kAdamWThreads) {
            float4 p = nt_load(P4 + i), m = nt_load(M4 + i), v = nt_load(V4 + i);
            adamw_vec(p, nt_load(G4 + i), m, v, c);
            nt_store(P4 + i, p);
            nt_store(M4 + i, m);
            nt_store(V4 + i, v);
        }
        scalar_from = nv << 2;
    }
    for (int e = scalar_from + tid; e < len; e += kAdamWThreads) {
        float p = P[e], m = M[e], v = V[e];
        adamw_elem(p, G[e], m, v, c);
        P[e] = p;
        M[e] = m;
        V[e] = v;
    }
}

__global__ __launch_bounds__(kAdamWThreads) void adamw_mt_kernel(const AdamWRec* __restrict__ recs,
                                                                  int n, AdamWConsts c) {
    const int64_t b = blockIdx.x;
    // Largest t with recs[t].block_begin <= b (block index is uniform: scalar loads).
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (recs[mid].block_begin <= b)
            lo = mid;
        else
            hi = mid - 1;
    }
    const AdamWRec r = recs[lo];
    const int64_t start = (b - r.block_begin) * kAdamWChunk;
    const int64_t rem = r.numel - start;
    adamw_chunk(r, start, rem < kAdamWChunk ? int(rem) : int(kAdamWChunk), c);
}

__global__ __launch_bounds__(kAdamWThreads) void adamw_one_kernel(AdamWRec r, AdamWConsts c) {
    const int64_t start = int64_t(blockIdx.x) * kAdamWChunk;
    const int64_t rem = r.numel - start;
    adamw_chunk(r, start, rem < kAdamWChunk ? int(rem) : int(kAdamWChunk), c);
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
    AdamWRec r;
    int st = adamw_table_pack(&t, 1, &r, sizeof(r), &blocks);
    if (st != MAMW_OK) return st;
    if (blocks == 0) return MAMW_OK;
    AdamWScalars s{lr, bias1, bias2, beta1, beta2, weight_decay, eps};
    return int(launch(K_ADAMW_ONE, 0, 0.0, 28.0 * double(numel), adamw_one_kernel, dim3(unsigned(blocks)),
                      dim3(kAdamWThreads), static_cast<hipStream_t>(stream), r, make_consts(s)));
}

extern "C" int mamw_adamw_table_bytes(int n_tensors, size_t* bytes) {
    return adamw_table_bytes(n_tensors, bytes);
}

extern "C" int mamw_adamw_table_pack(const mamw_adamw_tensor* tensors, int n_tensors,
                                     void* host_table, size_t table_bytes, int64_t* n_blocks) {
    return adamw_table_pack(tensors, n_tensors, host_table, table_bytes, n_blocks);
}

extern "C" int mamw_adamw_mt_step(const void* device_table, int n_tensors, int64_t n_blocks,
                                  float lr, float bias1, float bias2, float beta1, float beta2,
                                  float weight_decay, float eps, mamw_stream_t stream) {
    if (n_tensors < 0 || n_tensors > kMaxTensors) return MAMW_ERR_COUNT;
    if (n_blocks < 0 || n_blocks > int64_t(0x7fffffff)) return MAMW_ERR_NUMEL;
    if (n_blocks == 0) return MAMW_OK;
    if (n_tensors == 0) return MAMW_ERR_COUNT;
    if (!device_table) return MAMW_ERR_NULL;
    if (reinterpret_cast<uintptr_t>(device_table) % 16) return MAMW_ERR_ALIGN;
    AdamWScalars s{lr, bias1, bias2, beta1, beta2, weight_decay, eps};
    // Algorithmic bytes (28 per element) are not known here: the table is in device memory.
    return int(launch(K_ADAMW_MT, 0, 0.0, 0.0, adamw_mt_kernel, dim3(unsigned(n_blocks)), dim3(kAdamWThreads),
                      static_cast<hipStream_t>(stream), static_cast<const AdamWRec*>(device_table), n_tensors,
                      make_consts(s)));
}
