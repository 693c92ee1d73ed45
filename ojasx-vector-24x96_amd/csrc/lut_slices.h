// lut_slices.h -- the LUT slice loop shared by the many-instance kernels
// (grouped linears, routed experts): block_dim 16, 256 centroids, batch 1.
//
// A workgroup of NW waves owns R rows per thread of one instance.  For each
// 16-group slice s of the input it builds LUT_s[g][k] = <x[16(16s + g) ..], C[k]>
// (16 x 256 = X_s[16 x 16] . C^T[16 x 256]) with 64 fp32 MFMAs
// (v_mfma_f32_16x16x4f32; wave w computes the 16 / NW centroid tiles from
// (16 / NW) w), then each thread gathers the 16 entries its rows' codes
// select: 4 bytes of LDS per code byte.  Codes are slice-major tiles
// [S][Mp][16]: one 16-byte load per row and slice, PF slices in flight in a
// register ring, so a slice's gathers do not wait for HBM.
// With DB (two LUT buffers) the MFMAs of slice s + 1 are issued before the
// gathers of slice s and their results stored after them: one barrier per
// slice and the build off the critical path, for workgroups that are few per
// CU; with one buffer, build and gather alternate (two barriers per slice)
// and more workgroups fit a CU.
//
// MFMA 16x16x4 fp32 operand layout: lane l supplies A[m = l % 16][k = l / 16]
// and B[k = l / 16][n = l % 16]; the result's value v of lane l is
// D[m = 4 (l / 16) + v][n = l % 16].
#pragma once

#include "common.h"

namespace ojx {
namespace slices {

constexpr int kLutStride = 260;   // floats per LUT row (pads the MFMA stores' banks)
constexpr int kLutFloats = 16 * kLutStride;
typedef float v4f __attribute__((ext_vector_type(4)));

// LDS bytes of the LUT buffers.
constexpr size_t lut_bytes(bool db) { return (db ? 2 : 1) * kLutFloats * sizeof(float); }

// B operands of wave w: centroid tiles TPW w .. TPW w + TPW - 1 of the [256][16]
// codebook, bop[t][ks] = C[16 (TPW w + t) + lane % 16][4 ks + lane / 16].
template <int NW>
__device__ __forceinline__ void load_cb_operands(const float *__restrict__ cb, int w, int lane,
                                                 float (&bop)[16 / NW][4]) {
    constexpr int TPW = 16 / NW;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            bop[t][ks] = gld(cb + (16 * (TPW * w + t) + (lane & 15)) * 16 + 4 * ks + (lane >> 4));
}

__device__ __forceinline__ uint4 ld_code_row(const uint8_t *codes, int s, int Mp, int row) {
    return gld(reinterpret_cast<const uint4 *>(codes + ((size_t)s * Mp + row) * 16));
}

// Codes of slices s0 .. s0 + PF - 1 (slices from s1 on repeat s1 - 1 and go
// unused).  Every row index must be < Mp.
template <int PF, int R>
__device__ __forceinline__ void ring_start(const uint8_t *codes, const int (&row)[R], int Mp, int s0,
                                           int s1, uint4 (&ring)[PF][R]) {
#pragma unroll
    for (int q = 0; q < PF; ++q)
#pragma unroll
        for (int r = 0; r < R; ++r) ring[q][r] = ld_code_row(codes, min(s0 + q, s1 - 1), Mp, row[r]);
}

template <int NW>
__device__ __forceinline__ void build_issue(const float *xs, int s, int lane,
                                            const float (&bop)[16 / NW][4], v4f (&c)[16 / NW]) {
    constexpr int TPW = 16 / NW;
    float a[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) a[ks] = xs[s * 256 + (lane & 15) * 16 + 4 * ks + (lane >> 4)];
#pragma unroll
    for (int t = 0; t < TPW; ++t) c[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)       // the tiles' MFMA chains interleaved
#pragma unroll
        for (int t = 0; t < TPW; ++t)
            c[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[ks], bop[t][ks], c[t], 0, 0, 0);
}

template <int NW>
__device__ __forceinline__ void build_store(float *L, int w, int lane, const v4f (&c)[16 / NW]) {
    constexpr int TPW = 16 / NW;
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int v = 0; v < 4; ++v)
            L[(4 * (lane >> 4) + v) * kLutStride + 16 * (TPW * w + t) + (lane & 15)] = c[t][v];
}

template <int R>
__device__ __forceinline__ void gather(const float *L, const uint4 (&cw)[R], float (&acc)[R]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t wd[4] = {cw[r].x, cw[r].y, cw[r].z, cw[r].w};
        float pg[16];
#pragma unroll
        for (int g = 0; g < 16; ++g) pg[g] = L[g * kLutStride + ((wd[g >> 2] >> ((g & 3) * 8)) & 0xffu)];
        acc[r] += (((pg[0] + pg[1]) + (pg[2] + pg[3])) + ((pg[4] + pg[5]) + (pg[6] + pg[7]))) +
                  (((pg[8] + pg[9]) + (pg[10] + pg[11])) + ((pg[12] + pg[13]) + (pg[14] + pg[15])));
    }
}

// acc[r] += sum over slices s0 <= s < s1 of sum_g LUT_s[g][code(row r, s, g)],
// per slice a pairwise tree over the 16 groups, slices in order.  xs holds the
// input's slices (256 floats each, zero past the input length) and has been
// made visible by a barrier; L holds lut_bytes(DB).  Ends with a barrier.
template <int NW, int R, bool DB, int PF>
__device__ __forceinline__ void slice_loop(const float *xs, float *L, const float (&bop)[16 / NW][4],
                                           const uint8_t *codes, const int (&row)[R], int Mp, int s0,
                                           int s1, int w, int lane, uint4 (&ring)[PF][R],
                                           float (&acc)[R]) {
    constexpr int TPW = 16 / NW;
    v4f c[TPW];
    if constexpr (DB) {
        build_issue<NW>(xs, s0, lane, bop, c);
        build_store<NW>(L, w, lane, c);
        __syncthreads();
    }
    // Slice s uses ring slot q = (s - s0) % PF, a constant in the unrolled body,
    // so the ring never moves registers (a move of a register whose load is in
    // flight would wait for that load); the slot is refilled with slice s + PF
    // once its gathers are issued, unconditionally (past the last slice it
    // reloads that slice: a conditional load would need a second copy of the
    // slot).  With DB, slice s + 1's LUT is built unconditionally too (past the
    // last slice: a rebuild of it into the idle buffer, never read).  The main
    // loop runs whole groups of PF slices with no branch in its body, so the
    // wait counts for the ring stay exact across its back edge (a loop body with
    // several paths to its latch makes the compiler wait for every load in
    // flight at the loop head); the last (s1 - s0) % PF slices follow it.
    auto one = [&](const int s, const int q) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);   // each slice scheduled on its own
        if constexpr (DB) {
            build_issue<NW>(xs, min(s + 1, s1 - 1), lane, bop, c);
            gather(L + ((s - s0) & 1) * kLutFloats, ring[q], acc);
#pragma unroll
            for (int r = 0; r < R; ++r) ring[q][r] = ld_code_row(codes, min(s + PF, s1 - 1), Mp, row[r]);
            build_store<NW>(L + ((s + 1 - s0) & 1) * kLutFloats, w, lane, c);
            __syncthreads();   // slice s + 1's LUT written, slice s's gathers done
        } else {
            build_issue<NW>(xs, s, lane, bop, c);
            build_store<NW>(L, w, lane, c);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
            gather(L, ring[q], acc);
#pragma unroll
            for (int r = 0; r < R; ++r) ring[q][r] = ld_code_row(codes, min(s + PF, s1 - 1), Mp, row[r]);
            __syncthreads();   // the gathers of slice s before the build of s + 1
        }
    };
    int sb = s0;
    for (; sb + PF <= s1; sb += PF) {
#pragma unroll
        for (int q = 0; q < PF; ++q) one(sb + q, q);
    }
#pragma unroll
    for (int q = 0; q < PF - 1; ++q)
        if (sb + q < s1) one(sb + q, q);
}

}  // namespace slices
}  // namespace ojx
