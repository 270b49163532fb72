// Host-side planning and validation for the MuonAdamW kernels.
//
// Pure C++ (no HIP headers): everything here runs on the host before any HIP
// call, so argument errors surface as negative status codes on machines
// without a GPU as well.  The device records defined here are shared with the
// kernels (they include this header).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "muonadamw_amd.h"

namespace mamw {

// ---------------------------------------------------------------------------
// AdamW multi-tensor table.
//
// Device layout: n_tensors AdamWRec records (64 bytes each).  Launch block b
// belongs to the tensor t with rec[t].block_begin <= b < rec[t+1].block_begin
// (the block count closes the last range), and covers elements
// [(b - block_begin) * kAdamWChunk, +kAdamWChunk) of that tensor.
constexpr int kAdamWThreads = 256;
constexpr int kAdamWUnroll = 1;  // float4 groups per thread per block
constexpr int64_t kAdamWChunk = int64_t(kAdamWThreads) * 4 * kAdamWUnroll;  // 1024

struct alignas(16) AdamWRec {
    void* p;         // fp32, or bf16 with MAMW_BF16_PARAM
    const void* g;   // fp32, or bf16 with MAMW_BF16_GRAD
    float* m;
    float* v;
    int64_t numel;
    int64_t block_begin;
    int32_t vec_ok;  // every base pointer aligned for 4-element vector access
    int32_t flags;   // MAMW_BF16_* bits
    int32_t pad[2];
};
static_assert(sizeof(AdamWRec) == 64, "AdamWRec must stay 64 bytes");

struct AdamWScalars {
    float lr, bias1, bias2, beta1, beta2, weight_decay, eps;
};

int adamw_validate_tensor(const mamw_adamw_tensor_ex& t);
int adamw_table_bytes(int n_tensors, size_t* bytes);
int adamw_table_pack(const mamw_adamw_tensor* tensors, int n_tensors,
                     void* host_table, size_t table_bytes, int64_t* n_blocks);
int adamw_table_pack_ex(const mamw_adamw_tensor_ex* tensors, int n_tensors,
                        void* host_table, size_t table_bytes, int64_t* n_blocks);

// ---------------------------------------------------------------------------
// Muon batch plan.
//
// A batch holds matrices that share m = min(rows, cols) and n = max(rows, cols).
// Iterates live in the caller's workspace as zero-padded bf16 matrices:
//   X   [batch][mp][np]   the Newton-Schulz iterate (m x n), updated in place
//   XT0 [batch][np][mp]   its transpose (operand of B X), ping-pong with XT1
//   XT1 [batch][np][mp]   (only when ns_steps >= 2)
//   A   [batch][mp][mp]   Gram X X^T
//   B   [batch][mp][mp]   b A + c A A
//   part[batch][prep_tiles] fp32 partial sums of squares (one per prep unit)
//   inv [batch]           fp32 1 / max(bf16(||X||_F), eps)
constexpr int kPrepTile = 64;  // a prep unit holds kPrepTile^2 = 32 x 128 parameter elements
constexpr size_t kWsAlign = 256;

struct MuonMatDesc {
    float* param;
    const float* grad;
    float* mom;
    float* upd;  // optional orthogonalised-update output (NULL = skip)
    int64_t rows;
    int64_t cols;
    float slr;
    int32_t tall;   // rows > cols: X = bf16(u)^T
    int32_t flags;  // MAMW_BF16_* bits
};

struct MuonBatchDescs {
    MuonMatDesc d[MAMW_MUON_MAX_BATCH];
};

struct MuonPlan {
    int batch;
    int tile;  // GEMM tile edge (128 or 256); mp, np are multiples of it
    int64_t m, n, mp, np;
    int64_t prep_tiles;  // prep units, (mp/64) * (np/64); the prep kernel takes two per block
    int xkb;             // workspace matrices k-blocked: a whole matrix's byte offsets fit 31 bits
    // X is kept only when !xkb (the row-major Gram reads it); otherwise its
    // region is empty and off_x == off_xt0.
    size_t off_x, off_xt0, off_xt1, off_a, off_b, off_part, off_inv;
    size_t bytes;
};

int choose_tile(int64_t m, int64_t n, int batch);
int muon_plan(int batch, int64_t rows, int64_t cols, int ns_steps, MuonPlan* plan);
int muon_validate(const mamw_muon_matrix* mats, int batch, int ns_steps,
                  const void* workspace, size_t workspace_bytes, MuonPlan* plan,
                  MuonBatchDescs* descs);

// Limits (documented in the ABI through the error codes).
constexpr int64_t kMaxDim = int64_t(1) << 20;        // rows, cols <= 2^20
constexpr int64_t kMaxMatElems = int64_t(1) << 34;   // padded m*n per matrix
constexpr int64_t kMaxNumel = int64_t(1) << 40;      // AdamW elements per tensor
constexpr int kMaxTensors = 1 << 20;

// Byte ranges [a, a+na) and [b, b+nb) overlap (empty ranges never do).
bool ranges_overlap(const void* a, size_t na, const void* b, size_t nb);

inline int64_t round_up(int64_t x, int64_t to) { return (x + to - 1) / to * to; }
inline size_t align_ws(size_t x) { return (x + kWsAlign - 1) / kWsAlign * kWsAlign; }

}  // namespace mamw
