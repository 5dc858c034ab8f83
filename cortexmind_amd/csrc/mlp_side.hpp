// The MLP step's two short tails -- the output layer's finish (loss, b3, b2
// and W3 SGD steps from the fused head's per-workgroup partials) and the
// layer-1 bias step b1 -= lr * colsum(dH1) -- as work for the workgroups a
// paired weight-gradient launch adds on the CUs its two products leave free
// (gemm.hip: k_gemm_ring_pair).  They read only what the launch's products
// do not write, and write only what those do not read, so they run beside
// the products at no cost on the step's critical path; alone they were two
// more launches (about 11 us at the C5 shape).
//
// Head partial layout (mlp.hip, k_mlp_head): row p of `part` (one per head
// workgroup, `pw` floats) holds colsum dH2 [d2], then the loss sum and
// colsum dl [d3] in kHeadExtra floats, then gW3 [d3][d2].  Column sums over
// the rows run in k_head_finish's order: for each q in 0..15 the rows
// p = q, q + 16, ... in increasing p from 0, then the 16 sums in q order,
// so both kernels give the same bits.
#pragma once

#include "cxm_common.hpp"

namespace cxm {

constexpr int kHeadExtra = 32;  // head partial columns after gb2: the loss, then gb3 (padded)

struct StepSide {
    const float *part;  // head partials [blocks][pw], or null: no finish
    unsigned blocks, pw, d2, d3, b;
    float lr;
    float *loss, *b2, *b3, *w3;
    const float *dh1;  // [b, d1], 16-byte aligned, d1 % 4 == 0; null: no bias step
    float *b1;
    unsigned d1;
    unsigned wgs;  // side workgroups of the launch (0: none)
};

// Applies the finished sum g of head partial column col (k_head_finish's
// updates: two roundings for each SGD step).
__device__ __forceinline__ void head_col_apply(const StepSide &s, unsigned col, float g) {
    if (col < s.d2) {
        const float t = g * s.lr;
        s.b2[col] = s.b2[col] - t;
    } else if (col == s.d2) {
        s.loss[0] = g / static_cast<float>(s.b);
    } else if (col < s.d2 + kHeadExtra) {
        if (col - s.d2 - 1 < s.d3) {
            const float t = g * s.lr;
            s.b3[col - s.d2 - 1] = s.b3[col - s.d2 - 1] - t;
        }
    } else {
        const unsigned i = col - s.d2 - kHeadExtra, cls = i / s.d2, k = i - cls * s.d2;
        const float t = g * s.lr;
        s.w3[static_cast<size_t>(k) * s.d3 + cls] = s.w3[static_cast<size_t>(k) * s.d3 + cls] - t;
    }
}

// Side workgroup `wg` of s.wgs, 256 threads; `lds` holds 16 x 64 floats.
//  * finish: 64 columns per pass, four threads a column, thread qq summing
//    the rows of q = 4 qq .. 4 qq + 3 (16 loads in flight), the 16 q sums
//    then added in q order by one thread per column;
//  * bias: 64 columns per pass, thread (rp, cg) folding float4 column group
//    cg over rows rp, rp + 16, ... (16 loads in flight), the 16 row-phase
//    sums then added in rp order, and b1 -= sum * lr.
__device__ __forceinline__ void step_side(const StepSide &s, unsigned wg, float (*lds)[64]) {
    const int tid = threadIdx.x;
    if (s.part) {
        const int qq = tid & 3, c = tid >> 2;
        for (unsigned c0 = wg * 64; c0 < s.pw; c0 += s.wgs * 64) {
            const unsigned col = c0 + c;
            float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (col < s.pw) {
                const float *__restrict__ pc = s.part + col;
                for (unsigned p0 = 0; p0 < s.blocks; p0 += 64) {
                    float t[16];
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            // a clamped row, zeroed after: loads under a condition were
                            // compiled with a wait for each
                            const unsigned p = p0 + 16 * i + 4 * qq + j, pp = p < s.blocks ? p : s.blocks - 1;
                            t[4 * i + j] = pc[static_cast<size_t>(pp) * s.pw];
                        }
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            if (p0 + 16 * i + 4 * qq + j >= s.blocks) t[4 * i + j] = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
#pragma unroll
                        for (int j = 0; j < 4; ++j) v[j] += t[4 * i + j];  // past the last row: + 0, as k_head_finish
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) lds[4 * qq + j][c] = v[j];
            __syncthreads();
            if (tid < 64 && c0 + tid < s.pw) {
                float g = lds[0][tid];
#pragma unroll
                for (int q = 1; q < 16; ++q) g += lds[q][tid];
                head_col_apply(s, c0 + tid, g);
            }
            __syncthreads();
        }
    }
    if (s.dh1) {
        const int cg = tid & 15, rp = tid >> 4;
        for (unsigned c0 = wg * 64; c0 < s.d1; c0 += s.wgs * 64) {
            const unsigned col = c0 + 4 * cg;
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (col < s.d1) {
                const float *__restrict__ pc = s.dh1 + col;
                for (unsigned r0 = 0; r0 < s.b; r0 += 256) {
                    float4 t[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const unsigned r = r0 + rp + 16 * i, rr = r < s.b ? r : s.b - 1;
                        t[i] = ld4(pc + static_cast<size_t>(rr) * s.d1);
                    }
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        if (r0 + rp + 16 * i >= s.b) t[i] = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        a.x += t[i].x;
                        a.y += t[i].y;
                        a.z += t[i].z;
                        a.w += t[i].w;
                    }
                }
            }
            lds[rp][4 * cg] = a.x;
            lds[rp][4 * cg + 1] = a.y;
            lds[rp][4 * cg + 2] = a.z;
            lds[rp][4 * cg + 3] = a.w;
            __syncthreads();
            if (tid < 64 && c0 + tid < s.d1) {
                float g = lds[0][tid];
#pragma unroll
                for (int q = 1; q < 16; ++q) g += lds[q][tid];
                const float t = g * s.lr;
                s.b1[c0 + tid] = s.b1[c0 + tid] - t;
            }
            __syncthreads();
        }
    }
}

}  // namespace cxm
