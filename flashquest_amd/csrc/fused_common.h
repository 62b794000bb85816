// Helpers shared by the fused decode kernels (INT4 on the matrix cores,
// attn_mfma.hip, and TurboQuant, turbo_fused.hip): wave reductions, buffer
// loads through per-slice resources, and the in-kernel page scoring of one KV
// group (the arithmetic and fp32 order of score_kernel).
#pragma once

#include "select_common.h"

namespace fq {

constexpr int kMaxWgPages = 1024;           // pages of one workgroup split (entries staged in LDS)
constexpr int kSelC = 8;                    // in-kernel selection: pages per lane (P <= 512)

FQ_DEV float wave_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 32, 64));
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    v = fmaxf(v, dpp<kDppMirror>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppXor1>(v));
    return fmaxf(v, dpp<kDppXor2>(v));
}
FQ_DEV float row16_max(float v) {
    v = fmaxf(v, dpp<kDppMirror>(v));
    v = fmaxf(v, dpp<kDppHalfMirror>(v));
    v = fmaxf(v, dpp<kDppXor1>(v));
    return fmaxf(v, dpp<kDppXor2>(v));
}
FQ_DEV float lane_value(float v, int lane) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane)); }


FQ_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7FFFFFFF ? 0x7FFFFFFF : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}
FQ_DEV uint4 ld128(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
FQ_DEV uint32_t ld32(__amdgpu_buffer_rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
FQ_DEV uint2 ld64(__amdgpu_buffer_rsrc_t r, int off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2(v[0], v[1]);
}
FQ_DEV uint32_t ld16(__amdgpu_buffer_rsrc_t r, int off) { return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }


// Page scores of one KV group (P <= 64 * kSelC pages) by a whole workgroup of
// NT threads: 16 lanes per page, NT / 16 pages per pass.  score_group_load
// issues the metadata loads of the passes that hold pages (a partial last
// pass re-reads page P-1); score_group_regs scores them --
// score_kernel's arithmetic and order exactly -- and stores the sortable keys
// s_key[r * 64 kSelC + p] per query head, or (SUM, per_kv_head_sum) s_key[p]
// for the group's summed query, with 0 (below every score) for p >= P.
template <int NT>
struct ScoreRegs {
    static constexpr int kPass = 64 * kSelC / (NT / 16);
    uint4 sv[kPass], mv[kPass];
};

template <typename MT, int NT>
FQ_DEV void score_group_load(ScoreRegs<NT>& sr, const Int4Cache& c, int tid, int l, int b, int h) {
    constexpr int PPP = NT / 16;
    const int lip = tid & 15, pip = tid >> 4;
    const MT* ksc = (const MT*)c.ksc + l * c.ksc_s[0] + b * c.ksc_s[1] + h * c.ksc_s[2] + lip * 8;
    const MT* kmn = (const MT*)c.kmn + l * c.kmn_s[0] + b * c.kmn_s[1] + h * c.kmn_s[2] + lip * 8;
#pragma unroll
    for (int u = 0; u < ScoreRegs<NT>::kPass; ++u) {
        if (u * PPP < c.P) {          // uniform: no loads for passes past the group's pages
            const int p = min(u * PPP + pip, c.P - 1);
            sr.sv[u] = *(const uint4*)(ksc + p * 128);
            sr.mv[u] = *(const uint4*)(kmn + p * 128);
        }
    }
}

// Precomputed scores of one KV group (the workspace rows of score_kernel:
// `rows` rows of P fp32 scores) as the sortable keys of the in-kernel
// selection: s_key[r * 64 kSelC + p], 0 (below every score) for p >= P.
// scores_load issues the loads; scores_to_keys converts after they land.
template <int NREP, int NT>
struct ScoreRowRegs {
    static constexpr int kN = (NREP * 64 * kSelC + NT - 1) / NT;
    float v[kN];
};
template <int NREP, int NT>
FQ_DEV void scores_load(ScoreRowRegs<NREP, NT>& sr, const float* g_scores, int rows, int P, int tid) {
#pragma unroll
    for (int u = 0; u < ScoreRowRegs<NREP, NT>::kN; ++u) {
        const int i = tid + u * NT, r = i / (64 * kSelC), p = i % (64 * kSelC);
        sr.v[u] = g_scores[min(r, rows - 1) * P + min(p, P - 1)];
    }
}
template <int NREP, int NT>
FQ_DEV void scores_to_keys(const ScoreRowRegs<NREP, NT>& sr, uint32_t* s_key, int rows, int P, int tid) {
#pragma unroll
    for (int u = 0; u < ScoreRowRegs<NREP, NT>::kN; ++u) {
        const int i = tid + u * NT, r = i / (64 * kSelC), p = i % (64 * kSelC);
        if (r < rows) s_key[i] = p < P ? sortable_key(sr.v[u]) : 0u;
    }
}

// The page loop of the in-kernel scoring: NR rows of query values (qr) and
// their relu (qp), channels 8 * (tid & 15) .. + 7, against every page's
// metadata in registers; keys to s_key[r * 64 kSelC + p].
template <typename MT, int NR, int NT>
FQ_DEV void score_group_pages(const ScoreRegs<NT>& sr, const float (&qr)[NR][8], const float (&qp)[NR][8],
                              uint32_t* s_key, int tid, int P, float levels) {
    constexpr int PPP = NT / 16;
    const int lip = tid & 15, pip = tid >> 4;
#pragma unroll
    for (int u = 0; u < ScoreRegs<NT>::kPass; ++u) {
        const int p = u * PPP + pip;
        if (u * PPP < P) {            // uniform
            score_page_regs<NR, MT>(sr.sv[u], sr.mv[u], qr, qp, [&](int r, float sc) {
                if (lip == 0) s_key[r * 64 * kSelC + p] = p < P ? sortable_key(sc) : 0u;
            }, levels);
        } else if (lip == 0) {        // a pass past the group's pages: their keys are 0
#pragma unroll
            for (int r = 0; r < NR; ++r) s_key[r * 64 * kSelC + p] = 0u;
        }
    }
}

// qin[r][j]: query head r's raw value at channel 8 * (tid & 15) + j.
template <typename MT, int NREP, int NT, bool SUM>
FQ_DEV void score_group_regs_q(const ScoreRegs<NT>& sr, const float (&qin)[NREP][8], uint32_t* s_key, int tid, int P,
                               float levels = 15.0f) {
    // per_kv_head_sum scores the group's summed query, (q_0 + q_1) + ... with
    // relu applied per head before the sum; per_q_head scores every head
    constexpr int NR = SUM ? 1 : NREP;
    float qr[NR][8], qp[NR][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if constexpr (SUM) {
            float qs = qin[0][j];
            float ps = qs > 0.f ? qs : 0.f;
#pragma unroll
            for (int r = 1; r < NREP; ++r) {
                const float v = qin[r][j];
                qs = __fadd_rn(qs, v);
                ps = __fadd_rn(ps, v > 0.f ? v : 0.f);
            }
            qr[0][j] = qs;
            qp[0][j] = ps;
        } else {
#pragma unroll
            for (int r = 0; r < NREP; ++r) {
                qr[r][j] = qin[r][j];
                qp[r][j] = qr[r][j] > 0.f ? qr[r][j] : 0.f;
            }
        }
    }
    score_group_pages<MT, NR, NT>(sr, qr, qp, s_key, tid, P, levels);
}

// per_kv_head_sum over ROWS query heads read from LDS one row at a time
// (s_qraw[r][channel]): the summed query and the summed relu in
// score_group_regs_q's fp32 order, without every row's values live at once
// (the scoring registers hold the group's metadata loads meanwhile).
template <typename MT, int ROWS, int NT>
FQ_DEV void score_group_sum_lds(const ScoreRegs<NT>& sr, const float (*s_qraw)[128], uint32_t* s_key, int tid, int P,
                                float levels = 15.0f) {
    const int lip = tid & 15;
    float qr[1][8], qp[1][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float v = s_qraw[0][lip * 8 + j];
        qr[0][j] = v;
        qp[0][j] = v > 0.f ? v : 0.f;
    }
#pragma unroll 1
    for (int r = 1; r < ROWS; ++r) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = s_qraw[r][lip * 8 + j];
            qr[0][j] = __fadd_rn(qr[0][j], v);
            qp[0][j] = __fadd_rn(qp[0][j], v > 0.f ? v : 0.f);
        }
    }
    score_group_pages<MT, 1, NT>(sr, qr, qp, s_key, tid, P, levels);
}

template <typename MT, int NREP, int NT, bool SUM>
FQ_DEV void score_group_regs(const ScoreRegs<NT>& sr, const float (*s_qraw)[128], uint32_t* s_key, int tid, int P,
                             float levels = 15.0f) {
    const int lip = tid & 15;
    float qin[NREP][8];
#pragma unroll
    for (int r = 0; r < NREP; ++r)
#pragma unroll
        for (int j = 0; j < 8; ++j) qin[r][j] = s_qraw[r][lip * 8 + j];
    score_group_regs_q<MT, NREP, NT, SUM>(sr, qin, s_key, tid, P, levels);
}

}  // namespace fq
