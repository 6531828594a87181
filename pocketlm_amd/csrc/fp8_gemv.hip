// FP8 e4m3 block-scaled GEMV family for gfx950: linear, dual linear, SwiGLU
// MLP and the (weighted) many-expert MoE of src/pcketlm/native/fp8_linear.cpp.
//
// Design.  The path is HBM-bound (2 flop per weight byte at one activation
// row), so every kernel streams each weight byte once per call, for all
// activation rows, with 16-byte loads:
//
//   * A "chunk" is 1024 columns of one weight row: lane l of a wave reads
//     bytes [16l, 16l+16) with one global_load_dwordx4, decodes them with
//     v_cvt_pk_f32_fp8 (4 instructions per 16 bytes) and dots them with the
//     matching 16 activations.  The 16-byte span never crosses a 128-column
//     scale block, so the partial is scaled once.
//   * A workgroup owns a tile of TR rows and splits the row's chunks across
//     its waves (wave w takes chunks w, w+nw, ...); nw depends only on the
//     number of chunks per row, so the per-row arithmetic - lane partials,
//     the fixed xor-butterfly lane sum, the in-order sum over waves - is the
//     same for every batch size and tile shape.  That is what makes batched
//     calls bit-exact to per-row calls, as the reference's tests require.
//   * NaN weight bytes must contribute 0 (fp8_linear.cpp:31-33).  The fast
//     path decodes with the hardware converter (NaN stays NaN) and only when
//     a 16-byte partial comes out NaN re-decodes that span with NaN -> 0.
//
// fp8_rows_kernel  : rows of one or more experts sharing the activations
//                    (linear, dual, gate/up phase with the SiLU epilogue, and
//                    several weights of different row counts in one grid);
//                    the activations are fp32, or bf16 widened in the kernel
//                    (the *_bf16x_f32 entry points; widening is exact).
// fp8_combine_kernel: rows whose K range is the concatenation of several
//                    experts' down matrices, each with its own activations
//                    and route weight (down phase + routed combine); a last
//                    group can be split off into its own output (the shared
//                    expert beside the routed sum).
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <vector>

#include "common.h"
#include "route.h"

namespace {

constexpr int kMaxGroups = 64;  // experts per launch (pointer tables travel as kernel arguments)
constexpr int kMaxWaves = 8;
constexpr int kMaxM = 8;        // activation rows per launch; larger batches are split
constexpr int kMaxVar = 8;      // matrices of different row counts per many-linear launch

// Experts chosen on the device (the device-routed MoE).  moe_plan_kernel
// writes, for the sorted distinct experts of the router's [batch][top_k]
// indices, their six addresses (gate w/s, up w/s, down w/s; one row of tab
// per role) and the dense route matrix [group][batch].
constexpr int kPlanRoles = 6;
struct MoePlan {
    uint64_t tab[kPlanRoles][kMaxGroups];
    float route[kMaxGroups * kMaxM];
    int count;     // distinct accepted experts
    int pad[63];
};

struct RowsArgs {
    const uint8_t* w[2][kMaxGroups];
    const float* s[2][kMaxGroups];
    const float* x;       // activations [m_total][x_stride] (fp32), or
    const uint16_t* xb;   // the same as bf16 (non-null: read these; bf16 -> fp32 is exact)
    float* out[2];        // outputs, element (g, m, row) at ((g*m_total + m) * out_ld + row)
    int64_t x_stride;
    int64_t out_ld;
    int64_t rows;         // rows per group
    int64_t K;
    int64_t scale_cols;
    int tiles_per_group;
    int nchunks;
    int m_total;
    int m0;
    // Groups of different row counts (the many-linear entry point, one weight
    // per group): group g owns tiles [vtile[g], vtile[g+1]) of the grid and
    // writes its vrows[g] rows to vout[g] as [m_total][vrows[g]].  nvar = 0:
    // uniform groups as above.
    int nvar;
    int vtile[kMaxVar + 1];
    int64_t vrows[kMaxVar];
    float* vout[kMaxVar];
    // Device-chosen groups (the gate/up phase of the device-routed MoE):
    // group g < ndev takes its addresses from plan (tab rows 0-3), and only
    // the first plan->count of them run; group g >= ndev uses argument slot
    // g - ndev.  ndev = 0: all groups from the arguments.
    const MoePlan* plan;
    int ndev;
};

struct CombineArgs {
    const uint8_t* w[kMaxGroups];
    const float* s[kMaxGroups];
    const float* act;     // activations of group g: act + ((g_base+g)*m_total + m) * K
    const float* route;   // route of (g, m): route[(g_base+g)*route_sg + m*route_sm], or null (= 1)
    float* out;
    int64_t rows;
    int64_t K;
    int64_t scale_cols;
    int64_t route_sg;
    int64_t route_sm;
    int ngroups;
    int g_base;
    int cps;              // chunks per group segment
    int tiles_per_group;  // per_group_out only
    int per_group_out;    // 1: out[(g_base+g)*m_total + m][row]; 0: out[m][row] summed over groups
    int split_last;       // (summed mode) the last group is not summed: its own tiles write it, with
                          // route 1, to out_last[m][row]
    float* out_last;
    int accumulate;       // add to out instead of storing
    int zero_skip;        // skip (g, m) whose route is exactly 0
    int m_total;
    int m0;
    const MoePlan* plan;  // as in RowsArgs (tab rows 4-5 for the down matrices)
    int ndev;
    int fused;            // split_last computed inside the routed tiles (fp8_combine_kernel FUSED)
    uint16_t* out_bf16;   // fused only: bf16(bf16(out) + bf16(out_last)), or null
};

__device__ __forceinline__ float dot16(const float* w, const float* x) {
    float p = w[0] * x[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) p = fmaf(w[j], x[j], p);
    return p;
}

__device__ __forceinline__ void decode16(const uint4& q, float* w) {
    plm_decode4_e4m3(q.x, w);
    plm_decode4_e4m3(q.y, w + 4);
    plm_decode4_e4m3(q.z, w + 8);
    plm_decode4_e4m3(q.w, w + 12);
}

__device__ __forceinline__ void zero_nans16(float* w) {
#pragma unroll
    for (int j = 0; j < 16; ++j) w[j] = (w[j] != w[j]) ? 0.0f : w[j];
}

__device__ __forceinline__ void load_x16(const float* p, float* x) {
    const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = p4[i];
        x[4 * i + 0] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
    }
}

static_assert(kMaxGroups == 64, "the plan maps one lane of the first wave to each group");
struct PlanShared {
    int64_t key[64];
    float kw[64];
    int first[64];
    int64_t sel[kMaxGroups];
};

// Run by a whole workgroup (every thread calls it: it synchronises the
// workgroup); the first wave does the work.
__device__ void plan_from_choices(const uint64_t* __restrict__ table, int64_t num_experts, const int64_t* idx,
                                  const float* wts, int batch, int top_k, MoePlan* __restrict__ plan,
                                  int* __restrict__ rejected, PlanShared& ps) {
    const int lane = threadIdx.x;
    const bool w0 = lane < 64;
    const int n = batch * top_k;
    int64_t e = -1;
    uint64_t addr[kPlanRoles] = {0, 0, 0, 0, 0, 0};
    bool aligned = true, bad = false;
    if (w0) {
        // every load is issued before the first use: two memory round trips
        e = lane < n ? idx[lane] : -1;
        const float wj = lane < n ? wts[lane] : 0.0f;
        const bool in_range = e >= 0 && e < num_experts;
#pragma unroll
        for (int r = 0; r < kPlanRoles; ++r) addr[r] = in_range ? table[r * num_experts + e] : 0;
#pragma unroll
        for (int r = 0; r < kPlanRoles; ++r) aligned = aligned && (addr[r] & ((r & 1) ? 3u : 15u)) == 0;
        bad = lane < n && !(in_range && aligned);
        if (!in_range) e = -1;
        ps.key[lane] = e;
        ps.kw[lane] = wj;
    }
    __syncthreads();
    int f = 0;
    if (w0) {
        f = e >= 0;
        if (f)
            for (int i = 0; i < lane; ++i) f = f && ps.key[i] != e;
        ps.first[lane] = f;
    }
    __syncthreads();
    int count = 0;
    if (w0) {
        int rank = 0;
        for (int i = 0; i < n; ++i) {
            const int fi = ps.first[i];
            count += fi;
            rank += fi && ps.key[i] < e;
        }
        if (f) {
            ps.sel[rank] = e;
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r) plan->tab[r][rank] = aligned ? addr[r] : 0;
        }
        if (lane >= count) {
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r) plan->tab[r][lane] = 0;
        }
    }
    __syncthreads();
    if (w0) {
        for (int t = lane; t < kMaxGroups * batch; t += 64) {
            const int g = t / batch;
            const int m = t - g * batch;
            float w = 0.0f;
            if (g < count) {
                const int64_t want = ps.sel[g];
                for (int kk = top_k - 1; kk >= 0; --kk)  // the first of repeated choices wins
                    if (ps.key[m * top_k + kk] == want) w = ps.kw[m * top_k + kk];
            }
            plan->route[t] = w;
        }
        const unsigned long long badmask = __ballot(bad);
        if (lane == 0) {
            plan->count = count;
            if (rejected != nullptr) *rejected = __popcll(badmask);
        }
    }
}

// One wave (the whole workgroup) writes the plan of the router's
// n = batch * top_k choices (n <= 64) as run_fp8_moe builds it on the host
// (fp8_source.py:1600, 1653-1716): the distinct in-range experts in
// ascending order, their addresses from the device table [6][num_experts],
// and the route matrix [group][batch] (a row's weight for the expert, 0 when
// the row did not choose it; a repeated index within a row keeps its first
// weight).  An index outside [0, num_experts) is left out; an expert whose
// weight addresses are not 16-byte aligned (scales: 4) keeps its group but
// gets null addresses, so it contributes nothing.  Both are counted in
// *rejected.
__global__ __launch_bounds__(64) void moe_plan_kernel(const uint64_t* __restrict__ table, int64_t num_experts,
                                                      const int64_t* __restrict__ idx,
                                                      const float* __restrict__ wts, int batch, int top_k,
                                                      MoePlan* __restrict__ plan, int* __restrict__ rejected) {
    __shared__ PlanShared ps;
    plan_from_choices(table, num_experts, idx, wts, batch, top_k, plan, rejected, ps);
}

// The router and the plan in one launch: DeepSeek-V3 routing of every row's
// logits (route.h, the same choices and weights as ds_route_topk_f32), one
// wave per row, then the plan of those choices.  The choices and weights
// are also written to idx_out / w_out when those are not null.
//
// Up to 256 experts (4 per lane) the plan is built from registers: wave 0
// loads its lanes' rows of the expert table while the logits load, and the
// routing waves leave in LDS which of each lane's experts every row picked
// and with what weight.  The experts picked by any row, in ascending order,
// are then numbered by a prefix count over the lanes (the lanes hold
// ascending experts).  Wider tables go through plan_from_choices.
template <int J>
__global__ __launch_bounds__(512) void moe_route_plan_kernel(const float* __restrict__ logits,
                                                            const float* __restrict__ bias, int experts, int batch,
                                                            int top_k, int n_groups, int topk_groups, int scoring,
                                                            float route_scale, const uint64_t* __restrict__ table,
                                                            int64_t* idx_out, float* w_out,
                                                            MoePlan* __restrict__ plan, int* __restrict__ rejected) {
    extern __shared__ float4 sh4[];
    const int waves = static_cast<int>(blockDim.x >> 6);
    const int wave = static_cast<int>(threadIdx.x >> 6);
    const int lane = static_cast<int>(threadIdx.x & 63);
    const int e4 = (experts + 3) & ~3;
    float* route_lds = reinterpret_cast<float*>(sh4);  // [waves][2][e4]
    float* choice = route_lds + 2 * e4 * wave;
    float* score = choice + e4;
    __shared__ RouteWave rw[8];
    if constexpr (J == 4) {
        float* wdense = route_lds + 2 * e4 * waves;  // [batch][e4]: each row's weights, 0 where not picked
        __shared__ uint64_t picked[kMaxM][64];       // [row][lane]: bits of the lane's picked experts
        uint64_t tab[kPlanRoles][4];
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int e = 4 * lane + j;
                    tab[r][j] = e < experts ? table[static_cast<int64_t>(r) * experts + e] : 0;
                }
        }
        for (int m = wave; m < batch; m += waves)
            plm_route_wave<4>(logits + static_cast<int64_t>(m) * experts, bias, experts, top_k, n_groups, topk_groups,
                              scoring, route_scale, score, choice, rw[wave],
                              idx_out != nullptr ? idx_out + static_cast<int64_t>(m) * top_k : nullptr,
                              idx_out != nullptr ? w_out + static_cast<int64_t>(m) * top_k : nullptr, picked[m],
                              wdense + m * e4);
        __syncthreads();
        if (wave != 0) return;
        // every row's picks and weights of this lane's experts, read at once
        uint64_t pm[kMaxM];
        float4 wv[kMaxM];
        const bool owns = 4 * lane < experts;
#pragma unroll
        for (int m = 0; m < kMaxM; ++m) {
            pm[m] = m < batch ? picked[m][lane] : 0;
            wv[m] = m < batch && owns ? *reinterpret_cast<const float4*>(wdense + m * e4 + 4 * lane)
                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        uint64_t u = 0;
#pragma unroll
        for (int m = 0; m < kMaxM; ++m) u |= pm[m];
        const uint64_t below = (1ull << lane) - 1;
        int rank = 0, count = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t b = __ballot((u >> j) & 1ull);
            rank += __popcll(b & below);
            count += __popcll(b);
        }
        int bad = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (!((u >> j) & 1ull)) continue;
            bool aligned = true;
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r) aligned = aligned && (tab[r][j] & ((r & 1) ? 3u : 15u)) == 0;
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r) plan->tab[r][rank] = aligned ? tab[r][j] : 0;
#pragma unroll
            for (int m = 0; m < kMaxM; ++m) {
                if (m >= batch) break;
                plan->route[rank * batch + m] = reinterpret_cast<const float*>(&wv[m])[j];
                if (!aligned) bad += static_cast<int>((pm[m] >> j) & 1ull);
            }
            ++rank;
        }
        if (lane >= count) {
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r) plan->tab[r][lane] = 0;
            for (int m = 0; m < batch; ++m) plan->route[lane * batch + m] = 0.0f;
        }
        int total_bad = 0;  // bad <= 4 * kMaxM
#pragma unroll
        for (int bit = 0; bit < 6; ++bit) total_bad += __popcll(__ballot((bad >> bit) & 1)) << bit;
        if (lane == 0) {
            plan->count = count;
            if (rejected != nullptr) *rejected = total_bad;
        }
    } else {
        __shared__ PlanShared ps;
        __shared__ int64_t kidx[kMaxGroups];
        __shared__ float kwt[kMaxGroups];
        for (int m = wave; m < batch; m += waves)
            plm_route_wave<J>(logits + static_cast<int64_t>(m) * experts, bias, experts, top_k, n_groups, topk_groups,
                              scoring, route_scale, score, choice, rw[wave], kidx + m * top_k, kwt + m * top_k);
        __syncthreads();
        const int n = batch * top_k;
        if (idx_out != nullptr)
            for (int t = threadIdx.x; t < n; t += blockDim.x) {
                idx_out[t] = kidx[t];
                w_out[t] = kwt[t];
            }
        plan_from_choices(table, experts, kidx, kwt, batch, top_k, plan, rejected, ps);
    }
}

// 16 activations of row m at column col, from the fp32 or (XB) the bf16
// copy; both give the same fp32 values.
template <bool XB>
__device__ __forceinline__ void load_row_x16(const RowsArgs& a, int m, int64_t col, float* x) {
    const int64_t off = static_cast<int64_t>(a.m0 + m) * a.x_stride + col;
    if constexpr (XB) {
        const uint4* p = reinterpret_cast<const uint4*>(a.xb + off);
        const uint4 h0 = p[0], h1 = p[1];
        const uint32_t h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            x[2 * j] = __uint_as_float(h[j] << 16);
            x[2 * j + 1] = __uint_as_float(h[j] & 0xFFFF0000u);
        }
    } else {
        load_x16(a.x + off, x);
    }
}

template <int M, int TR, int NWT, bool SILU, bool XB>
__global__ __launch_bounds__(512) void fp8_rows_kernel(const RowsArgs a) {
    constexpr int V = NWT * TR * M;
    __shared__ float red[kMaxWaves * V];
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    int g;
    int64_t row0, rows = a.rows;
    if (a.nvar > 0) {
        g = 0;
        for (int i = 1; i < a.nvar; ++i)
            if (static_cast<int>(blockIdx.x) >= a.vtile[i]) g = i;
        row0 = static_cast<int64_t>(blockIdx.x - a.vtile[g]) * TR;
        rows = a.vrows[g];
    } else {
        g = blockIdx.x / a.tiles_per_group;
        row0 = static_cast<int64_t>(blockIdx.x - g * a.tiles_per_group) * TR;
    }

    const uint8_t* W[NWT];
    const float* S[NWT];
    int ga = g;  // argument slot
    if constexpr (NWT == 2 && SILU) {
        // (device-chosen groups exist only for the gate/up phase of the MoE)
        if (g < a.ndev) {
            if (g >= a.plan->count) return;  // the router chose fewer experts (uniform: before any barrier)
#pragma unroll
            for (int i = 0; i < NWT; ++i) {
                W[i] = reinterpret_cast<const uint8_t*>(a.plan->tab[2 * i][g]);
                S[i] = reinterpret_cast<const float*>(a.plan->tab[2 * i + 1][g]);
            }
        }
        ga = g - a.ndev;
    }
    if (ga >= 0) {
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            W[i] = a.w[i][ga];
            S[i] = a.s[i][ga];
        }
    }
    bool live = true;
#pragma unroll
    for (int i = 0; i < NWT; ++i) live = live && W[i] != nullptr && S[i] != nullptr;

    float acc[NWT][TR][M];
#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) acc[i][r][m] = 0.0f;

    if (live) {
        const int64_t srow = (row0 >> 7) * a.scale_cols;
        for (int c = wave; c < a.nchunks; c += nw) {
            const int64_t col = static_cast<int64_t>(c) * plm::kChunkBytes + lane * 16;
            if (col >= a.K) continue;
            // Loads are unconditional (rows past the end are clamped to the last
            // row and their results dropped) so that all of them issue before
            // the first wait.
            uint4 q[NWT][TR];
#pragma unroll
            for (int i = 0; i < NWT; ++i)
#pragma unroll
                for (int r = 0; r < TR; ++r) {
                    const int64_t rr = row0 + r < rows ? row0 + r : rows - 1;
                    q[i][r] = plm_gload16(W[i] + rr * a.K + col);
                }
            float sc[NWT];
#pragma unroll
            for (int i = 0; i < NWT; ++i) sc[i] = plm_gload_f32(S[i] + srow + (col >> 7));
            if constexpr (M == 1) {
                // one activation row: decode each weight row right before its
                // dot, so a larger tile needs no more registers (same arithmetic)
                float xv[16];
                load_row_x16<XB>(a, 0, col, xv);
#pragma unroll
                for (int i = 0; i < NWT; ++i)
#pragma unroll
                    for (int r = 0; r < TR; ++r) {
                        float w16[16];
                        decode16(q[i][r], w16);
                        float p = dot16(w16, xv);
                        if (p != p) {
                            zero_nans16(w16);
                            p = dot16(w16, xv);
                        }
                        acc[i][r][0] = fmaf(p, sc[i], acc[i][r][0]);
                    }
                continue;
            }
            if constexpr (TR >= 8) {
                // wide tiles with several activation rows: each weight row is
                // decoded again for every activation row (registers for one
                // decoded row only), halving the activation reads per weight
                // byte; a NaN span is redone with NaN bytes as 0, which equals
                // using the sanitised row for every activation row.
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float xv[16];
                    load_row_x16<XB>(a, m, col, xv);
#pragma unroll
                    for (int i = 0; i < NWT; ++i)
#pragma unroll
                        for (int r = 0; r < TR; ++r) {
                            // opaque copy: the compiler would otherwise keep
                            // every decoded row live across the activation rows
                            uint4 qq = q[i][r];
                            asm volatile("" : "+v"(qq.x), "+v"(qq.y), "+v"(qq.z), "+v"(qq.w));
                            float w16[16];
                            decode16(qq, w16);
                            float p = dot16(w16, xv);
                            if (p != p) {
                                zero_nans16(w16);
                                p = dot16(w16, xv);
                            }
                            acc[i][r][m] = fmaf(p, sc[i], acc[i][r][m]);
                        }
                }
                continue;
            }
            float wv[NWT][TR][16];
#pragma unroll
            for (int i = 0; i < NWT; ++i)
#pragma unroll
                for (int r = 0; r < TR; ++r) decode16(q[i][r], wv[i][r]);
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float xv[16];
                load_row_x16<XB>(a, m, col, xv);
#pragma unroll
                for (int i = 0; i < NWT; ++i)
#pragma unroll
                    for (int r = 0; r < TR; ++r) {
                        float p = dot16(wv[i][r], xv);
                        if (m == 0 && p != p) {
                            zero_nans16(wv[i][r]);
                            p = dot16(wv[i][r], xv);
                        }
                        acc[i][r][m] = fmaf(p, sc[i], acc[i][r][m]);
                    }
            }
        }
    }

#pragma unroll
    for (int i = 0; i < NWT; ++i)
#pragma unroll
        for (int r = 0; r < TR; ++r)
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float t = plm_wave_sum(acc[i][r][m]);
                if (lane == kSumLane) red[wave * V + (i * TR + r) * M + m] = t;
            }
    __syncthreads();

    for (int t = threadIdx.x; t < TR * M; t += blockDim.x) {
        const int r = t / M;
        const int m = t - r * M;
        const int64_t row = row0 + r;
        if (row >= rows) continue;
        float v[NWT];
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[w * V + (i * TR + r) * M + m];
            v[i] = s;
        }
        const int64_t o = (static_cast<int64_t>(g) * a.m_total + a.m0 + m) * a.out_ld + row;
        if constexpr (SILU) {
            a.out[0][o] = plm_silu_mul(v[0], v[1]);
        } else {
            if (a.nvar > 0) {
                a.vout[g][static_cast<int64_t>(a.m0 + m) * rows + row] = v[0];
                continue;
            }
#pragma unroll
            for (int i = 0; i < NWT; ++i) a.out[i][o] = v[i];
        }
    }
}

// bf16 bits of v rounded to nearest even (finite and infinite v).
__device__ __forceinline__ uint32_t bf16_rne_bits(float v) {
    const uint32_t b = __float_as_uint(v);
    return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_value(float v) { return v != v ? v : __uint_as_float(bf16_rne_bits(v) << 16); }

// The reference's bf16 tail of the MoE (fp8_source.py:1597, 1762, 1861-1862),
// done by torch on the host there: a bf16 tensor of zeros, plus
// routed.to(bf16), plus shared.to(bf16).  Each bf16 add is an fp32 add
// rounded to nearest even, and a NaN sum comes out as 0x7FC0.
__device__ __forceinline__ uint16_t moe_bf16_tail(float routed, float shared, bool has_shared) {
    float v = 0.0f + bf16_value(routed);  // exact; -0 becomes +0 as in zeros + x
    if (has_shared) v = v + bf16_value(shared);
    return static_cast<uint16_t>(v != v ? 0x7FC0u : bf16_rne_bits(v));
}

// One (group g, chunk cc) item of the down phase for a tile of TR rows:
// acc[r][m] += route(g, m) * scale * (D_g[row0 + r, chunk] . act_g,m[chunk]).
template <int M, int TR>
__device__ __forceinline__ void combine_chunk(const CombineArgs& a, int g, int cc, bool weighted, int64_t row0,
                                              int lane, float (&acc)[TR][M]) {
    const int64_t col = static_cast<int64_t>(cc) * plm::kChunkBytes + lane * 16;
    const uint8_t* W;
    const float* S;
    if (g < a.ndev) {
        W = reinterpret_cast<const uint8_t*>(a.plan->tab[4][g]);
        S = reinterpret_cast<const float*>(a.plan->tab[5][g]);
    } else {
        W = a.w[g - a.ndev];
        S = a.s[g - a.ndev];
    }
    if (W == nullptr || S == nullptr) return;
    float rw[M];
    bool any = false;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        rw[m] = a.route && weighted ? a.route[static_cast<int64_t>(a.g_base + g) * a.route_sg +
                                              static_cast<int64_t>(a.m0 + m) * a.route_sm]
                                    : 1.0f;
        any = any || !(a.zero_skip && rw[m] == 0.0f);
    }
    if (!any || col >= a.K) return;
    uint4 q[TR];
#pragma unroll
    for (int r = 0; r < TR; ++r) {
        const int64_t rr = row0 + r < a.rows ? row0 + r : a.rows - 1;
        q[r] = plm_gload16(W + rr * a.K + col);
    }
    const float sc = plm_gload_f32(S + (row0 >> 7) * a.scale_cols + (col >> 7));
    if constexpr (M == 1) {
        // one activation row: decode each weight row right before its dot,
        // so a larger tile needs no more registers (same arithmetic)
        if (a.zero_skip && rw[0] == 0.0f) return;
        float xv[16];
        load_x16(a.act + (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0) * a.K + col, xv);
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            float w16[16];
            decode16(q[r], w16);
            float p = dot16(w16, xv);
            if (p != p) {
                zero_nans16(w16);
                p = dot16(w16, xv);
            }
            acc[r][0] = fmaf(p * sc, rw[0], acc[r][0]);
        }
        return;
    }
    float wv[TR][16];
#pragma unroll
    for (int r = 0; r < TR; ++r) decode16(q[r], wv[r]);
    bool fixed = false;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if (a.zero_skip && rw[m] == 0.0f) continue;
        float xv[16];
        load_x16(a.act + (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0 + m) * a.K + col, xv);
#pragma unroll
        for (int r = 0; r < TR; ++r) {
            float p = dot16(wv[r], xv);
            if (!fixed && p != p) {
                zero_nans16(wv[r]);
                p = dot16(wv[r], xv);
            }
            acc[r][m] = fmaf(p * sc, rw[m], acc[r][m]);
        }
        fixed = true;
    }
}

// FUSED (the device-routed MoE): one workgroup computes both the routed sum
// and the split-off last group (the shared expert) of its rows, each with
// the item-to-wave assignment of the split tiles, and also writes the bf16
// tail of the two when out_bf16 is set.
template <int M, int TR, bool FUSED>
__global__ __launch_bounds__(512) void fp8_combine_kernel(const CombineArgs a) {
    constexpr int V = TR * M;
    __shared__ float red[(FUSED ? 2 : 1) * kMaxWaves * V];
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    int g_lo = 0;
    int g_hi = a.ngroups;
    int tile = blockIdx.x;
    bool last = false;  // this workgroup computes the split-off last group
    if (a.per_group_out) {
        g_lo = tile / a.tiles_per_group;
        g_hi = g_lo + 1;
        tile -= g_lo * a.tiles_per_group;
    } else if (a.split_last) {
        g_hi = a.ngroups - 1;
        if (!FUSED && tile >= a.tiles_per_group) {
            tile -= a.tiles_per_group;
            g_lo = g_hi;
            g_hi = a.ngroups;
            last = true;
        }
    }
    const int64_t row0 = static_cast<int64_t>(tile) * TR;
    // Device-chosen groups past the router's count are left out.  The items
    // before them keep their wave assignment (item c goes to wave c % nw), so
    // the sums are those of a call given just the chosen groups.
    if (a.ndev > 0 && !last) g_hi = min(g_hi, a.plan->count);

    float acc[TR][M];
#pragma unroll
    for (int r = 0; r < TR; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;

    const int nchunks = (g_hi - g_lo) * a.cps;
    for (int c = wave; c < nchunks; c += nw) {
        const int gi = c / a.cps;
        combine_chunk<M, TR>(a, g_lo + gi, c - gi * a.cps, !last, row0, lane, acc);
    }
#pragma unroll
    for (int r = 0; r < TR; ++r)
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float t = plm_wave_sum(acc[r][m]);
            if (lane == kSumLane) red[wave * V + r * M + m] = t;
        }
    if constexpr (FUSED) {
        // The split-off group in the same registers.  With fewer items than
        // waves its items go, in order, to the last waves (those with the
        // fewest routed items), one each: the wave sums then add the same
        // values in the same order as a tile of its own (whose item c sits
        // on wave c), the other waves adding exact zeros.
        if (a.split_last) {
#pragma unroll
            for (int r = 0; r < TR; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) acc[r][m] = 0.0f;
            const int shift = nw > a.cps ? nw - a.cps : 0;
            for (int c = wave - shift; c < a.cps; c += nw)
                if (c >= 0) combine_chunk<M, TR>(a, a.ngroups - 1, c, false, row0, lane, acc);
#pragma unroll
            for (int r = 0; r < TR; ++r)
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float t = plm_wave_sum(acc[r][m]);
                    if (lane == kSumLane) red[(kMaxWaves + wave) * V + r * M + m] = t;
                }
        }
    }
    __syncthreads();

    for (int t = threadIdx.x; t < V; t += blockDim.x) {
        const int r = t / M;
        const int m = t - r * M;
        const int64_t row = row0 + r;
        if (row >= a.rows) continue;
        float v = 0.0f;
        for (int w = 0; w < nw; ++w) v += red[w * V + t];
        int64_t o = static_cast<int64_t>(a.m0 + m) * a.rows + row;
        if constexpr (FUSED) {
            float v2 = 0.0f;
            if (a.split_last) {
                for (int w = 0; w < nw; ++w) v2 += red[(kMaxWaves + w) * V + t];
                a.out_last[o] = v2;
            }
            a.out[o] = v;
            if (a.out_bf16 != nullptr) a.out_bf16[o] = moe_bf16_tail(v, v2, a.split_last != 0);
        } else {
            if (a.per_group_out) o += static_cast<int64_t>(a.g_base + g_lo) * a.m_total * a.rows;
            float* dst = last ? a.out_last : a.out;
            dst[o] = a.accumulate ? dst[o] + v : v;
        }
    }
}

// ----------------------------------------------------------------- scalar path
// Used when K is not a multiple of 16 or a pointer is not 16-byte aligned
// (small test shapes).  One thread per output element; the per-row arithmetic
// is again independent of the batch size.

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// x is fp32, or bf16 when xb is non-null.
__device__ float scalar_row_dot(const uint8_t* w, const float* s, const float* x, int64_t K,
                                const uint16_t* xb = nullptr) {
    float acc = 0.0f;
    for (int64_t c0 = 0; c0 < K; c0 += 128) {
        const int64_t c1 = c0 + 128 < K ? c0 + 128 : K;
        float blk = 0.0f;
        for (int64_t c = c0; c < c1; ++c) {
            const uint32_t byte = w[c];
            float v[4];
            plm_decode4_e4m3(byte, v);
            const float wv = (v[0] != v[0]) ? 0.0f : v[0];
            blk = fmaf(xb != nullptr ? bf16_bits_to_f32(xb[c]) : x[c], wv, blk);
        }
        acc = fmaf(blk, s[c0 >> 7], acc);
    }
    return acc;
}

template <bool SILU, int NWT>
__global__ void fp8_rows_scalar_kernel(const RowsArgs a, int mcount, int ngroups) {
    const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t total = static_cast<int64_t>(ngroups) * mcount * a.rows;
    if (id >= total) return;
    const int64_t row = id % a.rows;
    const int m = static_cast<int>((id / a.rows) % mcount);
    const int g = static_cast<int>(id / (a.rows * mcount));
    float v[NWT];
    for (int i = 0; i < NWT; ++i) {
        const uint8_t* W = a.w[i][g];
        const float* S = a.s[i][g];
        if (W == nullptr || S == nullptr) {
            v[i] = 0.0f;
            continue;
        }
        const int64_t xo = static_cast<int64_t>(a.m0 + m) * a.x_stride;
        v[i] = scalar_row_dot(W + row * a.K, S + (row >> 7) * a.scale_cols, a.x + xo, a.K,
                              a.xb != nullptr ? a.xb + xo : nullptr);
    }
    bool live = true;
    for (int i = 0; i < NWT; ++i) live = live && a.w[i][g] != nullptr && a.s[i][g] != nullptr;
    const int64_t o = (static_cast<int64_t>(g) * a.m_total + a.m0 + m) * a.out_ld + row;
    if constexpr (SILU) {
        a.out[0][o] = live ? plm_silu_mul(v[0], v[1]) : 0.0f;
    } else {
        for (int i = 0; i < NWT; ++i) a.out[i][o] = v[i];
    }
}

__global__ void fp8_combine_scalar_kernel(const CombineArgs a, int mcount) {
    const int64_t id = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int ng_out = a.per_group_out ? a.ngroups : (a.split_last ? 2 : 1);
    const int64_t total = static_cast<int64_t>(ng_out) * mcount * a.rows;
    if (id >= total) return;
    const int64_t row = id % a.rows;
    const int m = static_cast<int>((id / a.rows) % mcount);
    const int go = static_cast<int>(id / (a.rows * mcount));
    const bool last = !a.per_group_out && a.split_last && go == 1;
    const int g_lo = a.per_group_out ? go : (last ? a.ngroups - 1 : 0);
    const int g_hi = a.per_group_out ? go + 1 : (a.split_last && !last ? a.ngroups - 1 : a.ngroups);
    float v = 0.0f;
    for (int g = g_lo; g < g_hi; ++g) {
        const uint8_t* W = a.w[g];
        const float* S = a.s[g];
        if (W == nullptr || S == nullptr) continue;
        const float rw = a.route && !last ? a.route[static_cast<int64_t>(a.g_base + g) * a.route_sg +
                                                    static_cast<int64_t>(a.m0 + m) * a.route_sm]
                                          : 1.0f;
        if (a.zero_skip && rw == 0.0f) continue;
        const float e = scalar_row_dot(W + row * a.K, S + (row >> 7) * a.scale_cols,
                                       a.act + (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0 + m) * a.K,
                                       a.K);
        v = fmaf(e, rw, v);
    }
    int64_t o = static_cast<int64_t>(a.m0 + m) * a.rows + row;
    if (a.per_group_out) o += static_cast<int64_t>(a.g_base + go) * a.m_total * a.rows;
    float* dst = last ? a.out_last : a.out;
    dst[o] = a.accumulate ? dst[o] + v : v;
}

__global__ void fill_f32_kernel(float* p, float v, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// The dense route matrix [E, M] of sparse (item, row, weight) pairs: one
// thread per cell adds the weights of its pairs in pair order (as the
// reference's sequential scatter does), so no zero fill and no atomics.
// Pairs with an index out of range match no cell; with bad set, workgroup 0
// also counts them into *bad (one writer).
__global__ __launch_bounds__(256) void scatter_pairs_kernel(const int64_t* items, const int64_t* rows, const float* w,
                                                            int64_t pairs, int64_t experts, int64_t batch,
                                                            float* route, int* bad) {
    const int64_t cell = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (cell < experts * batch) {
        const int64_t e = cell / batch, r = cell - e * batch;
        float v = 0.0f;
        for (int64_t p = 0; p < pairs; ++p)
            if (items[p] == e && rows[p] == r) v += w[p];
        route[cell] = v;
    }
    if (bad != nullptr && blockIdx.x == 0) {
        __shared__ int count;
        if (threadIdx.x == 0) count = 0;
        __syncthreads();
        int n = 0;
        for (int64_t p = threadIdx.x; p < pairs; p += blockDim.x)
            n += items[p] < 0 || items[p] >= experts || rows[p] < 0 || rows[p] >= batch;
        if (n) atomicAdd(&count, n);
        __syncthreads();
        if (threadIdx.x == 0) *bad = count;
    }
}


// ------------------------------------------------------------------ dispatch

int waves_for(int64_t nchunks) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(nchunks, kMaxWaves)));
}

// Rows per tile.  The per-row arithmetic does not depend on it, so it is
// chosen per launch: at one or two activation rows (where each weight row is
// decoded right before its dot) 8 rows halve the activation reads per weight
// byte, used when the grid still has at least kTileWaves waves; otherwise 4
// for one weight, and 2 for two (gate and up): measured on the DeepSeek-V3
// gate/up launch (9 x 2 weights of 2048 x 7168, M = 1) at 45.4 us with 2-row
// tiles against 47.3 us with 4-row ones (twice the workgroups, the same
// bytes per wave).
constexpr int64_t kTileWaves = 4096;

template <int M>
constexpr int rows_tile(int nwt) {
    return nwt == 1 ? 4 : 2;
}

template <int M>
constexpr int combine_tile() {
    return 4;
}

bool wide_tile_fits(int64_t rows, int64_t groups, int nw) {
    return plm::ceil_div(rows, 8) * groups * nw >= kTileWaves;
}

// With one weight, halving the tile to 2 rows pays when 4-row tiles would
// leave CUs idle (fewer tiles than CUs) or load them unevenly (the busiest
// CU's share of ceil(tiles / CUs) is above the mean by more than it would be
// with twice the tiles): 1536 rows give 384 tiles of 4, 1.5 per CU, against
// 768 of 2, 3 per CU.  Where both divide evenly (2048, 3072 rows) the
// 4-row tile reads the activations half as often and stays.
bool narrow_tile_balances(int64_t tiles4) {
    const int64_t cus = plm::cu_count();
    const int64_t tiles2 = 2 * tiles4;
    return tiles4 < cus || plm::ceil_div(tiles2, cus) * tiles4 < plm::ceil_div(tiles4, cus) * tiles2;
}

template <int M, int TR, int NWT, bool SILU>
void launch_rows_tr(const RowsArgs& a, int ngroups, hipStream_t st) {
    RowsArgs b = a;
    b.tiles_per_group = static_cast<int>(plm::ceil_div(a.rows, TR));
    const int nw = waves_for(a.nchunks);
    int64_t grid = static_cast<int64_t>(b.tiles_per_group) * ngroups;
    if (a.nvar > 0) {
        b.vtile[0] = 0;
        for (int i = 0; i < a.nvar; ++i)
            b.vtile[i + 1] = b.vtile[i] + static_cast<int>(plm::ceil_div(a.vrows[i], TR));
        grid = b.vtile[a.nvar];
    }
    if (a.xb != nullptr) {
        hipLaunchKernelGGL((fp8_rows_kernel<M, TR, NWT, SILU, true>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    } else {
        hipLaunchKernelGGL((fp8_rows_kernel<M, TR, NWT, SILU, false>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    }
}

template <int M, int NWT, bool SILU>
void launch_rows_m(const RowsArgs& a, int ngroups, hipStream_t st) {
    if constexpr (NWT == 1) {
        int64_t all_rows = a.rows;
        int64_t tiles4 = plm::ceil_div(a.rows, 4) * ngroups;
        if (a.nvar > 0) {
            all_rows = 0;
            tiles4 = 0;
            for (int i = 0; i < a.nvar; ++i) {
                all_rows += a.vrows[i];
                tiles4 += plm::ceil_div(a.vrows[i], 4);
            }
        }
        // (at three or more activation rows the wide tile's re-decoding and
        // registers cost more than the activation reads it saves)
        if constexpr (M <= 2) {
            if (wide_tile_fits(all_rows, a.nvar > 0 ? 1 : ngroups, waves_for(a.nchunks))) {
                launch_rows_tr<M, 8, 1, SILU>(a, ngroups, st);
                return;
            }
        }
        if (narrow_tile_balances(tiles4)) {
            launch_rows_tr<M, 2, 1, SILU>(a, ngroups, st);
            return;
        }
    }
    launch_rows_tr<M, rows_tile<M>(NWT), NWT, SILU>(a, ngroups, st);
}

template <int NWT, bool SILU>
void launch_rows(const RowsArgs& a, int mcount, int ngroups, hipStream_t st) {
    switch (mcount) {
        case 1: launch_rows_m<1, NWT, SILU>(a, ngroups, st); break;
        case 2: launch_rows_m<2, NWT, SILU>(a, ngroups, st); break;
        case 3: launch_rows_m<3, NWT, SILU>(a, ngroups, st); break;
        case 4: launch_rows_m<4, NWT, SILU>(a, ngroups, st); break;
        case 5: launch_rows_m<5, NWT, SILU>(a, ngroups, st); break;
        case 6: launch_rows_m<6, NWT, SILU>(a, ngroups, st); break;
        case 7: launch_rows_m<7, NWT, SILU>(a, ngroups, st); break;
        default: launch_rows_m<8, NWT, SILU>(a, ngroups, st); break;
    }
}

// Groups summed by one output tile: every group in summed mode, except a
// split-off last group, whose own tiles (one group each) read it on the same
// wave split.  Tiles of one output per group in per_group_out mode.
int combine_segments(const CombineArgs& a) {
    return a.per_group_out ? 1 : (a.split_last ? a.ngroups - 1 : a.ngroups);
}

int combine_outputs(const CombineArgs& a) {
    return a.per_group_out ? a.ngroups : (a.split_last && !a.fused ? 2 : 1);
}

template <int M, int TR>
void launch_combine_tr(const CombineArgs& a, hipStream_t st) {
    CombineArgs b = a;
    const int tiles = static_cast<int>(plm::ceil_div(a.rows, TR));
    b.tiles_per_group = tiles;
    const int nw = waves_for(combine_segments(a) * a.cps);
    const int64_t grid = static_cast<int64_t>(tiles) * combine_outputs(a);
    if (a.fused) {
        hipLaunchKernelGGL((fp8_combine_kernel<M, TR, true>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    } else {
        hipLaunchKernelGGL((fp8_combine_kernel<M, TR, false>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    }
}

template <int M>
void launch_combine_m(const CombineArgs& a, hipStream_t st) {
    if constexpr (M == 1) {
        // (fused tiles also carry the split-off group: 4-row tiles keep the
        // grid at several workgroups per CU)
        if (wide_tile_fits(a.rows, combine_outputs(a), waves_for(combine_segments(a) * a.cps))) {
            launch_combine_tr<1, 8>(a, st);
            return;
        }
    }
    launch_combine_tr<M, combine_tile<M>()>(a, st);
}

void launch_combine(const CombineArgs& a, int mcount, hipStream_t st) {
    switch (mcount) {
        case 1: launch_combine_m<1>(a, st); break;
        case 2: launch_combine_m<2>(a, st); break;
        case 3: launch_combine_m<3>(a, st); break;
        case 4: launch_combine_m<4>(a, st); break;
        case 5: launch_combine_m<5>(a, st); break;
        case 6: launch_combine_m<6>(a, st); break;
        case 7: launch_combine_m<7>(a, st); break;
        default: launch_combine_m<8>(a, st); break;
    }
}

// A GEMV problem over groups that share the activations.
struct RowsProblem {
    const uint8_t* const* w[2];  // per-group pointers, ngroups entries each
    const float* const* s[2];
    int nwt;
    bool silu;
    int ngroups;
    const float* x;
    const uint16_t* xb;   // bf16 activations instead of x (one of the two is set)
    int64_t x_stride;
    float* out[2];
    int64_t out_ld;
    int64_t batch;
    int64_t rows;
    int64_t K;
    int64_t scale_cols;
    int nvar;             // > 0: ngroups single weights of vrows[g] rows each, written to vout[g]
    int64_t vrows[kMaxVar];
    float* vout[kMaxVar];
};

bool rows_fast_ok(const RowsProblem& p) {
    if (p.xb != nullptr) {
        if (p.K % 16 != 0 || p.x_stride % 8 != 0 || !plm::aligned16(p.xb)) return false;
    } else if (p.K % 16 != 0 || p.x_stride % 4 != 0 || !plm::aligned16(p.x)) {
        return false;
    }
    for (int i = 0; i < p.nwt; ++i)
        for (int g = 0; g < p.ngroups; ++g)
            if (!plm::aligned16(p.w[i][g])) return false;
    return true;
}

int run_rows(const RowsProblem& p, hipStream_t st) {
    const bool fast = rows_fast_ok(p);
    if (p.nvar > 0 && (!fast || p.nwt != 1 || p.ngroups != p.nvar || p.nvar > kMaxVar))
        return plm::fail(-2, "variable-row groups need the vector path and one weight per group");
    for (int g0 = 0; g0 < p.ngroups; g0 += kMaxGroups) {
        const int ng = std::min(kMaxGroups, p.ngroups - g0);
        RowsArgs a;
        std::memset(&a, 0, sizeof(a));
        for (int i = 0; i < p.nwt; ++i)
            for (int g = 0; g < ng; ++g) {
                a.w[i][g] = p.w[i][g0 + g];
                a.s[i][g] = p.s[i][g0 + g];
            }
        a.x = p.x;
        a.xb = p.xb;
        a.x_stride = p.x_stride;
        // Output offsets of this group batch: element (g, m, row) lives at
        // ((g0 + g) * batch + m) * out_ld + row.
        for (int i = 0; i < p.nwt; ++i) {
            a.out[i] = p.out[i] ? p.out[i] + static_cast<int64_t>(g0) * p.batch * p.out_ld : nullptr;
        }
        a.out_ld = p.out_ld;
        a.rows = p.rows;
        a.K = p.K;
        a.scale_cols = p.scale_cols;
        a.nchunks = static_cast<int>(plm::ceil_div(p.K, plm::kChunkBytes));
        a.m_total = static_cast<int>(p.batch);
        a.nvar = p.nvar;
        for (int i = 0; i < p.nvar; ++i) {
            a.vrows[i] = p.vrows[i];
            a.vout[i] = p.vout[i];
        }
        for (int64_t m0 = 0; m0 < p.batch; m0 += kMaxM) {
            const int mc = static_cast<int>(std::min<int64_t>(kMaxM, p.batch - m0));
            a.m0 = static_cast<int>(m0);
            if (fast) {
                if (p.nwt == 1) {
                    launch_rows<1, false>(a, mc, ng, st);
                } else if (p.silu) {
                    launch_rows<2, true>(a, mc, ng, st);
                } else {
                    launch_rows<2, false>(a, mc, ng, st);
                }
            } else {
                const int64_t total = static_cast<int64_t>(ng) * mc * p.rows;
                const unsigned blocks = static_cast<unsigned>(plm::ceil_div(total, 256));
                if (p.nwt == 1) {
                    hipLaunchKernelGGL((fp8_rows_scalar_kernel<false, 1>), dim3(blocks), dim3(256), 0, st, a, mc, ng);
                } else if (p.silu) {
                    hipLaunchKernelGGL((fp8_rows_scalar_kernel<true, 2>), dim3(blocks), dim3(256), 0, st, a, mc, ng);
                } else {
                    hipLaunchKernelGGL((fp8_rows_scalar_kernel<false, 2>), dim3(blocks), dim3(256), 0, st, a, mc, ng);
                }
            }
            const int code = plm::check_launch("fp8 rows kernel");
            if (code != 0) return code;
        }
    }
    return 0;
}

// Down phase: out[m][row] = sum_g route(g, m) * (D_g . act_g,m)[row], or one
// output per group when per_group_out.
struct CombineProblem {
    const uint8_t* const* w;
    const float* const* s;
    int ngroups;
    const float* act;     // [ngroups][batch][K]
    const float* route;   // see route_sg / route_sm, or null
    int64_t route_sg;
    int64_t route_sm;
    bool zero_skip;
    bool per_group_out;
    float* out;
    float* out_last;      // summed mode: the last group is left out of the sum and written here, route 1
    int64_t batch;
    int64_t rows;
    int64_t K;
    int64_t scale_cols;
};

int run_combine(const CombineProblem& p, hipStream_t st) {
    if (p.out_last != nullptr && (p.per_group_out || p.ngroups < 2 || p.ngroups > kMaxGroups))
        return plm::fail(-2, "a split-off last group needs 2..%d summed groups", kMaxGroups);
    bool fast = p.K % 16 == 0 && plm::aligned16(p.act);
    for (int g = 0; g < p.ngroups && fast; ++g) fast = plm::aligned16(p.w[g]);
    for (int g0 = 0; g0 < p.ngroups; g0 += kMaxGroups) {
        const int ng = std::min(kMaxGroups, p.ngroups - g0);
        CombineArgs a;
        std::memset(&a, 0, sizeof(a));
        for (int g = 0; g < ng; ++g) {
            a.w[g] = p.w[g0 + g];
            a.s[g] = p.s[g0 + g];
        }
        a.act = p.act;
        a.route = p.route;
        a.route_sg = p.route_sg;
        a.route_sm = p.route_sm;
        a.out = p.out;
        a.rows = p.rows;
        a.K = p.K;
        a.scale_cols = p.scale_cols;
        a.ngroups = ng;
        a.g_base = g0;
        a.cps = static_cast<int>(plm::ceil_div(p.K, plm::kChunkBytes));
        a.per_group_out = p.per_group_out ? 1 : 0;
        a.split_last = p.out_last != nullptr ? 1 : 0;
        a.out_last = p.out_last;
        a.accumulate = (!p.per_group_out && g0 > 0) ? 1 : 0;
        a.zero_skip = p.zero_skip ? 1 : 0;
        a.m_total = static_cast<int>(p.batch);
        for (int64_t m0 = 0; m0 < p.batch; m0 += kMaxM) {
            const int mc = static_cast<int>(std::min<int64_t>(kMaxM, p.batch - m0));
            a.m0 = static_cast<int>(m0);
            if (fast) {
                launch_combine(a, mc, st);
            } else {
                const int64_t total = static_cast<int64_t>(combine_outputs(a)) * mc * p.rows;
                const unsigned blocks = static_cast<unsigned>(plm::ceil_div(total, 256));
                hipLaunchKernelGGL(fp8_combine_scalar_kernel, dim3(blocks), dim3(256), 0, st, a, mc);
            }
            const int code = plm::check_launch("fp8 combine kernel");
            if (code != 0) return code;
        }
    }
    return 0;
}

int fill_f32(float* p, float v, int64_t n, hipStream_t st) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(fill_f32_kernel, dim3(static_cast<unsigned>(plm::ceil_div(n, 256))), dim3(256), 0, st,
                       p, v, n);
    return plm::check_launch("fill kernel");
}

// Gather six host address tables into typed vectors.
struct ExpertTables {
    std::vector<const uint8_t*> g, u, d;
    std::vector<const float*> gs, us, ds;
    ExpertTables(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp,
                 const uint64_t* dp, const uint64_t* dsp, int64_t n) {
        for (int64_t e = 0; e < n; ++e) {
            g.push_back(reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(gp[e])));
            gs.push_back(reinterpret_cast<const float*>(static_cast<uintptr_t>(gsp[e])));
            u.push_back(reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(up[e])));
            us.push_back(reinterpret_cast<const float*>(static_cast<uintptr_t>(usp[e])));
            d.push_back(reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(dp[e])));
            ds.push_back(reinterpret_cast<const float*>(static_cast<uintptr_t>(dsp[e])));
        }
    }
};

// Activations as the caller passed them: fp32, or bf16 (the bf16 twins of
// the entry points; bf16 -> fp32 is exact, so both give the same results).
struct Act {
    const float* f32;
    const uint16_t* bf16;
};

// Phase 1 of every SwiGLU path: act[e][m][row] = silu(gate_e . x_m) * (up_e . x_m).
int gate_up_phase(const ExpertTables& t, int64_t experts, Act hidden, float* act,
                  int64_t batch, int64_t inter, int64_t hid, int64_t gsc, hipStream_t st) {
    RowsProblem p;
    std::memset(&p, 0, sizeof(p));
    p.w[0] = t.g.data();
    p.w[1] = t.u.data();
    p.s[0] = t.gs.data();
    p.s[1] = t.us.data();
    p.nwt = 2;
    p.silu = true;
    p.ngroups = static_cast<int>(experts);
    p.x = hidden.f32;
    p.xb = hidden.bf16;
    p.x_stride = hid;
    p.out[0] = act;
    p.out[1] = nullptr;
    p.out_ld = inter;
    p.batch = batch;
    p.rows = inter;
    p.K = hid;
    p.scale_cols = gsc;
    return run_rows(p, st);
}

bool moe_dims_bad(int64_t experts, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    return experts <= 0 || batch <= 0 || inter <= 0 || hid <= 0 || gsc < plm::ceil_div(hid, 128) ||
           dsc < plm::ceil_div(inter, 128);
}

// Shared body of the weighted / row-weighted MoE entry points.
// With out_last, the tables hold one more expert after the `experts` routed
// ones: it runs in the same two launches and is written, unweighted, to
// out_last instead of joining the routed sum.
int weighted_moe(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp,
                 const uint64_t* dp, const uint64_t* dsp, Act hidden, const float* route,
                 int64_t route_sg, int64_t route_sm, bool zero_skip, float* out, int64_t experts,
                 int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc, float* out_last = nullptr) {
    hipStream_t st = plm::current_stream();
    const int64_t groups = experts + (out_last != nullptr ? 1 : 0);
    float* act = static_cast<float*>(plm::workspace(static_cast<size_t>(groups * batch * inter) * sizeof(float)));
    if (act == nullptr) return -3;
    ExpertTables t(gp, gsp, up, usp, dp, dsp, groups);
    int code = gate_up_phase(t, groups, hidden, act, batch, inter, hid, gsc, st);
    if (code != 0) return code;
    CombineProblem c;
    std::memset(&c, 0, sizeof(c));
    c.w = t.d.data();
    c.s = t.ds.data();
    c.ngroups = static_cast<int>(groups);
    c.act = act;
    c.route = route;
    c.route_sg = route_sg;
    c.route_sm = route_sm;
    c.zero_skip = zero_skip;
    c.per_group_out = false;
    c.out = out;
    c.out_last = out_last;
    c.batch = batch;
    c.rows = hid;
    c.K = inter;
    c.scale_cols = dsc;
    return run_combine(c, st);
}

int linear_impl(const uint8_t* fp8_weight, const float* scale_inv, Act hidden, float* out, int64_t batch,
                int64_t out_rows, int64_t in_cols, int64_t scale_cols) {
    if (batch <= 0 || out_rows <= 0 || in_cols <= 0 || scale_cols < plm::ceil_div(in_cols, 128))
        return plm::fail(-2, "bad dimensions");
    const uint8_t* w[1] = {fp8_weight};
    const float* s[1] = {scale_inv};
    RowsProblem p;
    std::memset(&p, 0, sizeof(p));
    p.w[0] = w;
    p.s[0] = s;
    p.nwt = 1;
    p.ngroups = 1;
    p.x = hidden.f32;
    p.xb = hidden.bf16;
    p.x_stride = in_cols;
    p.out[0] = out;
    p.out_ld = out_rows;
    p.batch = batch;
    p.rows = out_rows;
    p.K = in_cols;
    p.scale_cols = scale_cols;
    return run_rows(p, plm::current_stream());
}

int dual_linear_impl(const uint8_t* wa, const float* sa, const uint8_t* wb, const float* sb, Act hidden,
                     float* out_a, float* out_b, int64_t batch, int64_t out_rows, int64_t in_cols,
                     int64_t scale_cols) {
    if (batch <= 0 || out_rows <= 0 || in_cols <= 0 || scale_cols < plm::ceil_div(in_cols, 128))
        return plm::fail(-2, "bad dimensions");
    const uint8_t* w0[1] = {wa};
    const uint8_t* w1[1] = {wb};
    const float* s0[1] = {sa};
    const float* s1[1] = {sb};
    RowsProblem p;
    std::memset(&p, 0, sizeof(p));
    p.w[0] = w0;
    p.w[1] = w1;
    p.s[0] = s0;
    p.s[1] = s1;
    p.nwt = 2;
    p.silu = false;
    p.ngroups = 1;
    p.x = hidden.f32;
    p.xb = hidden.bf16;
    p.x_stride = in_cols;
    p.out[0] = out_a;
    p.out[1] = out_b;
    p.out_ld = out_rows;
    p.batch = batch;
    p.rows = out_rows;
    p.K = in_cols;
    p.scale_cols = scale_cols;
    return run_rows(p, plm::current_stream());
}

int mlp_impl(const uint8_t* gate_weight, const float* gate_scale_inv, const uint8_t* up_weight,
             const float* up_scale_inv, const uint8_t* down_weight, const float* down_scale_inv, Act hidden,
             float* out, int64_t batch, int64_t intermediate_rows, int64_t hidden_cols, int64_t gate_scale_cols,
             int64_t down_scale_cols) {
    if (moe_dims_bad(1, batch, intermediate_rows, hidden_cols, gate_scale_cols, down_scale_cols))
        return plm::fail(-2, "bad dimensions");
    const uint64_t gp = reinterpret_cast<uintptr_t>(gate_weight), gsp = reinterpret_cast<uintptr_t>(gate_scale_inv);
    const uint64_t upp = reinterpret_cast<uintptr_t>(up_weight), usp = reinterpret_cast<uintptr_t>(up_scale_inv);
    const uint64_t dp = reinterpret_cast<uintptr_t>(down_weight), dsp = reinterpret_cast<uintptr_t>(down_scale_inv);
    hipStream_t st = plm::current_stream();
    float* act = static_cast<float*>(plm::workspace(static_cast<size_t>(batch * intermediate_rows) * sizeof(float)));
    if (act == nullptr) return -3;
    ExpertTables t(&gp, &gsp, &upp, &usp, &dp, &dsp, 1);
    int code = gate_up_phase(t, 1, hidden, act, batch, intermediate_rows, hidden_cols, gate_scale_cols, st);
    if (code != 0) return code;
    CombineProblem c;
    std::memset(&c, 0, sizeof(c));
    c.w = t.d.data();
    c.s = t.ds.data();
    c.ngroups = 1;
    c.act = act;
    c.out = out;
    c.batch = batch;
    c.rows = hidden_cols;
    c.K = intermediate_rows;
    c.scale_cols = down_scale_cols;
    return run_combine(c, st);
}

// bad_pairs null: the reference's contract, indices checked on the host
// (read back, so the call synchronises its stream) and -4 for one out of
// range.  bad_pairs set: no host read-back; pairs out of range are left out
// and counted into *bad_pairs (device memory), so the call never waits.
int pair_weighted_impl(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp,
                       const uint64_t* dp, const uint64_t* dsp, Act hidden, const int64_t* pair_item_indices,
                       const int64_t* pair_row_indices, const float* pair_weights, float* out, int64_t expert_count,
                       int64_t pair_count, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc,
                       int* bad_pairs = nullptr) {
    if (pair_count < 0 || moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc))
        return plm::fail(-2, "bad dimensions");
    hipStream_t st = plm::current_stream();
    int code = fill_f32(out, 0.0f, batch * hid, st);
    if (code != 0) return code;
    if (pair_count == 0) {
        if (bad_pairs != nullptr) {
            hipLaunchKernelGGL(scatter_pairs_kernel, dim3(1), dim3(256), 0, st, pair_item_indices, pair_row_indices,
                               pair_weights, int64_t(0), int64_t(0), batch, static_cast<float*>(nullptr), bad_pairs);
            return plm::check_launch("scatter pairs");
        }
        return 0;
    }
    if (bad_pairs == nullptr) {
        // The index check needs the values on the host: read them back.
        std::vector<int64_t> items(static_cast<size_t>(pair_count)), rows(static_cast<size_t>(pair_count));
        hipError_t err = hipMemcpyAsync(items.data(), pair_item_indices, sizeof(int64_t) * pair_count,
                                        hipMemcpyDeviceToHost, st);
        if (err == hipSuccess)
            err = hipMemcpyAsync(rows.data(), pair_row_indices, sizeof(int64_t) * pair_count, hipMemcpyDeviceToHost,
                                 st);
        if (err == hipSuccess) err = hipStreamSynchronize(st);
        if (err != hipSuccess) return plm::hip_fail(err, "pair index read-back");
        for (int64_t p = 0; p < pair_count; ++p) {
            if (items[p] < 0 || items[p] >= expert_count || rows[p] < 0 || rows[p] >= batch)
                return plm::fail(-4, "pair %lld out of range", static_cast<long long>(p));
        }
    }
    // Dense route matrix [E, batch] after the activations in the workspace.
    const size_t act_elems = static_cast<size_t>(expert_count * batch * inter);
    float* ws = static_cast<float*>(plm::workspace((act_elems + static_cast<size_t>(expert_count * batch)) * sizeof(float)));
    if (ws == nullptr) return -3;
    float* route = ws + act_elems;
    const int64_t cells = std::max<int64_t>(expert_count * batch, 1);
    hipLaunchKernelGGL(scatter_pairs_kernel, dim3(static_cast<unsigned>(plm::ceil_div(cells, 256))), dim3(256), 0, st,
                       pair_item_indices, pair_row_indices, pair_weights, pair_count, expert_count, batch, route,
                       bad_pairs);
    code = plm::check_launch("scatter pairs");
    if (code != 0) return code;
    // weighted_moe asks for the same workspace size prefix, so act stays at ws.
    ExpertTables t(gp, gsp, up, usp, dp, dsp, expert_count);
    code = gate_up_phase(t, expert_count, hidden, ws, batch, inter, hid, gsc, st);
    if (code != 0) return code;
    CombineProblem c;
    std::memset(&c, 0, sizeof(c));
    c.w = t.d.data();
    c.s = t.ds.data();
    c.ngroups = static_cast<int>(expert_count);
    c.act = ws;
    c.route = route;
    c.route_sg = batch;
    c.route_sm = 1;
    c.zero_skip = true;
    c.out = out;
    c.batch = batch;
    c.rows = hid;
    c.K = inter;
    c.scale_cols = dsc;
    return run_combine(c, st);
}

// The MoE with the experts chosen on the device: the router's indices and
// weights stay in HBM.  A one-wave kernel writes the plan (the chosen
// experts' addresses out of a device table of all experts, and the route
// matrix) that the gate/up and down launches read.  Same values as the host-routed calls given the same experts
// in ascending order (the weighted call at batch 1, the row-weighted one
// above it; with a shared expert, its merged form), the shared expert and
// the bf16 tail computed by the down launch's workgroups.
// fixed: a block the caller provides (fixed_bytes long) instead of the
// library's workspace, for the entry point that allocates nothing.
// Routing done in the same launch as the plan: the router's logits and
// settings (ds_route_topk_f32's arguments).  idx / wts then receive the
// choices and weights (when not null) instead of providing them.
struct RouteFromLogits {
    const float* logits;
    const float* bias;
    int n_groups;
    int topk_groups;
    int scoring;
    float route_scale;
};

int device_routed_impl(const uint64_t* table, int64_t num_experts, const int64_t* idx, const float* wts,
                       int64_t top_k, const uint64_t* shared, Act hidden, float* out, float* out_shared,
                       uint16_t* out_bf16, int* rejected, int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                       int64_t dsc, char* fixed = nullptr, size_t fixed_bytes = 0,
                       const RouteFromLogits* route = nullptr) {
    if (num_experts <= 0 || num_experts > INT32_MAX || top_k <= 0 || batch <= 0 || batch > kMaxM ||
        batch * top_k > kMaxGroups)
        return plm::fail(-2, "bad dimensions (batch 1..%d, batch * top_k <= %d)", kMaxM, kMaxGroups);
    if (moe_dims_bad(1, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    const void* x = hidden.f32 != nullptr ? static_cast<const void*>(hidden.f32) : static_cast<const void*>(hidden.bf16);
    if (hid % 16 != 0 || inter % 16 != 0 || !plm::aligned16(x))
        return plm::fail(-2, "device routing needs sizes that are multiples of 16 and 16-byte aligned activations");
    if (shared != nullptr) {
        for (int r = 0; r < kPlanRoles; ++r)
            if (shared[r] == 0) return plm::fail(-1, "null pointer");
        if ((shared[0] | shared[2] | shared[4]) & 15u) return plm::fail(-2, "shared expert weights must be 16-byte aligned");
    }
    hipStream_t st = plm::current_stream();
    const int ndev = static_cast<int>(batch * top_k);
    const int groups = ndev + (shared != nullptr ? 1 : 0);
    const size_t act_bytes =
        static_cast<size_t>(plm::ceil_div(static_cast<int64_t>(groups) * batch * inter * 4, 256) * 256);
    char* ws;
    if (fixed != nullptr) {
        if (act_bytes + sizeof(MoePlan) > fixed_bytes)
            return plm::fail(-2, "the call needs %zu bytes of scratch, more than the %zu this entry point holds",
                             act_bytes + sizeof(MoePlan), fixed_bytes);
        ws = fixed;
    } else {
        ws = static_cast<char*>(plm::workspace(act_bytes + sizeof(MoePlan)));
        if (ws == nullptr) return -3;
    }
    float* act = reinterpret_cast<float*>(ws);
    MoePlan* plan = reinterpret_cast<MoePlan*>(ws + act_bytes);
    if (route != nullptr) {
        // one wave per row while the per-wave arrays fit 32 KiB
        const int64_t e4 = (num_experts + 3) & ~int64_t(3);
        const int64_t per_wave = 2 * e4 * static_cast<int64_t>(sizeof(float));
        const int waves = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(batch, 32768 / per_wave)));
        const int j = plm_route_j(static_cast<int>(num_experts));
        const size_t shmem =
            static_cast<size_t>(per_wave * waves + (j == 4 ? batch * e4 * static_cast<int64_t>(sizeof(float)) : 0));
        auto kern = j == 4 ? moe_route_plan_kernel<4> : (j == 16 ? moe_route_plan_kernel<16> : moe_route_plan_kernel<64>);
        hipLaunchKernelGGL(kern, dim3(1), dim3(64 * waves), shmem, st, route->logits, route->bias,
                           static_cast<int>(num_experts), static_cast<int>(batch), static_cast<int>(top_k),
                           route->n_groups, route->topk_groups, route->scoring, route->route_scale, table,
                           const_cast<int64_t*>(idx), const_cast<float*>(wts), plan, rejected);
    } else {
        hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(64), 0, st, table, num_experts, idx, wts,
                           static_cast<int>(batch), static_cast<int>(top_k), plan, rejected);
    }
    int code = plm::check_launch("moe plan kernel");
    if (code != 0) return code;

    RowsArgs a;
    std::memset(&a, 0, sizeof(a));
    if (shared != nullptr) {
        a.w[0][0] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(shared[0]));
        a.s[0][0] = reinterpret_cast<const float*>(static_cast<uintptr_t>(shared[1]));
        a.w[1][0] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(shared[2]));
        a.s[1][0] = reinterpret_cast<const float*>(static_cast<uintptr_t>(shared[3]));
    }
    a.x = hidden.f32;
    a.xb = hidden.bf16;
    a.x_stride = hid;
    a.out[0] = act;
    a.out_ld = inter;
    a.rows = inter;
    a.K = hid;
    a.scale_cols = gsc;
    a.nchunks = static_cast<int>(plm::ceil_div(hid, plm::kChunkBytes));
    a.m_total = static_cast<int>(batch);
    a.plan = plan;
    a.ndev = ndev;
    launch_rows<2, true>(a, static_cast<int>(batch), groups, st);
    code = plm::check_launch("fp8 rows kernel");
    if (code != 0) return code;

    CombineArgs c;
    std::memset(&c, 0, sizeof(c));
    if (shared != nullptr) {
        c.w[0] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(shared[4]));
        c.s[0] = reinterpret_cast<const float*>(static_cast<uintptr_t>(shared[5]));
    }
    c.act = act;
    c.route = reinterpret_cast<const float*>(reinterpret_cast<const char*>(plan) + offsetof(MoePlan, route));
    c.route_sg = batch;
    c.route_sm = 1;
    c.zero_skip = batch > 1 ? 1 : 0;
    c.out = out;
    c.split_last = shared != nullptr ? 1 : 0;
    c.out_last = shared != nullptr ? out_shared : nullptr;
    c.rows = hid;
    c.K = inter;
    c.scale_cols = dsc;
    c.ngroups = groups;
    c.cps = static_cast<int>(plm::ceil_div(inter, plm::kChunkBytes));
    c.m_total = static_cast<int>(batch);
    c.plan = plan;
    c.ndev = ndev;
    c.fused = 1;
    c.out_bf16 = out_bf16;
    launch_combine(c, static_cast<int>(batch), st);
    return plm::check_launch("fp8 combine kernel");
}

// Several weights of different row counts sharing the activations, in one
// launch when the vector path applies (else one call per weight; the per-row
// arithmetic is the same either way).
int linear_many_impl(const uint64_t* weight_ptrs, const uint64_t* scale_ptrs, Act hidden, const uint64_t* out_ptrs,
                     const int64_t* out_rows, int64_t count, int64_t batch, int64_t in_cols, int64_t scale_cols) {
    if (count <= 0 || count > kMaxVar) return plm::fail(-2, "1..%d weights per call", kMaxVar);
    if (batch <= 0 || in_cols <= 0 || scale_cols < plm::ceil_div(in_cols, 128)) return plm::fail(-2, "bad dimensions");
    const uint8_t* w[kMaxVar];
    const float* s[kMaxVar];
    RowsProblem p;
    std::memset(&p, 0, sizeof(p));
    int64_t max_rows = 0;
    for (int64_t i = 0; i < count; ++i) {
        w[i] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(weight_ptrs[i]));
        s[i] = reinterpret_cast<const float*>(static_cast<uintptr_t>(scale_ptrs[i]));
        p.vout[i] = reinterpret_cast<float*>(static_cast<uintptr_t>(out_ptrs[i]));
        p.vrows[i] = out_rows[i];
        if (!w[i] || !s[i] || !p.vout[i]) return plm::fail(-1, "null pointer");
        if (out_rows[i] <= 0) return plm::fail(-2, "bad dimensions");
        max_rows = std::max(max_rows, out_rows[i]);
    }
    p.w[0] = w;
    p.s[0] = s;
    p.nwt = 1;
    p.ngroups = static_cast<int>(count);
    p.nvar = static_cast<int>(count);
    p.x = hidden.f32;
    p.xb = hidden.bf16;
    p.x_stride = in_cols;
    p.batch = batch;
    p.rows = max_rows;
    p.K = in_cols;
    p.scale_cols = scale_cols;
    if (rows_fast_ok(p)) return run_rows(p, plm::current_stream());
    for (int64_t i = 0; i < count; ++i) {
        const int code = linear_impl(w[i], s[i], hidden, p.vout[i], batch, out_rows[i], in_cols, scale_cols);
        if (code != 0) return code;
    }
    return 0;
}

}  // namespace

// ------------------------------------------------------- allocation-free entry point
// fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc keeps its scratch (the
// activations and the plan) in this array instead of the library's
// workspace, so it never allocates.  Each device holds its own copy for the
// life of the process; every call on a device shares it.
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(8) << 20;  // 8 MiB
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_dev[kMaxDevices] = {};  // the array's device address, per device

// The array's address on the current device, looked up the first time a
// device calls (with that device current) and kept.  In host code the
// array's name is not a device address: only this pointer is passed on.
int scratch_address(char** out) {
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return plm::hip_fail(err, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return plm::fail(-2, "device %d beyond the %d this library tracks", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess) return plm::hip_fail(err, "hipGetSymbolAddress(scratch)");
        g_scratch_dev[dev] = static_cast<char*>(p);
    }
    *out = g_scratch_dev[dev];
    return 0;
}

}  // namespace

// ====================================================================== C ABI

PLM_EXPORT int fp8_e4m3_block_linear_f32(const uint8_t* fp8_weight, const float* scale_inv,
                                         const float* hidden, float* out, int64_t batch,
                                         int64_t out_rows, int64_t in_cols, int64_t scale_cols) {
    if (!fp8_weight || !scale_inv || !hidden || !out) return plm::fail(-1, "null pointer");
    return linear_impl(fp8_weight, scale_inv, Act{hidden, nullptr}, out, batch, out_rows, in_cols, scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_linear_bf16x_f32(const uint8_t* fp8_weight, const float* scale_inv,
                                               const uint16_t* hidden_bf16, float* out, int64_t batch,
                                               int64_t out_rows, int64_t in_cols, int64_t scale_cols) {
    if (!fp8_weight || !scale_inv || !hidden_bf16 || !out) return plm::fail(-1, "null pointer");
    return linear_impl(fp8_weight, scale_inv, Act{nullptr, hidden_bf16}, out, batch, out_rows, in_cols, scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_linear_many_f32(const uint64_t* weight_ptrs, const uint64_t* scale_ptrs,
                                              const float* hidden, const uint64_t* out_ptrs, const int64_t* out_rows,
                                              int64_t count, int64_t batch, int64_t in_cols, int64_t scale_cols) {
    if (!weight_ptrs || !scale_ptrs || !hidden || !out_ptrs || !out_rows) return plm::fail(-1, "null pointer");
    return linear_many_impl(weight_ptrs, scale_ptrs, Act{hidden, nullptr}, out_ptrs, out_rows, count, batch, in_cols,
                            scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_linear_many_bf16x_f32(const uint64_t* weight_ptrs, const uint64_t* scale_ptrs,
                                                    const uint16_t* hidden_bf16, const uint64_t* out_ptrs,
                                                    const int64_t* out_rows, int64_t count, int64_t batch,
                                                    int64_t in_cols, int64_t scale_cols) {
    if (!weight_ptrs || !scale_ptrs || !hidden_bf16 || !out_ptrs || !out_rows) return plm::fail(-1, "null pointer");
    return linear_many_impl(weight_ptrs, scale_ptrs, Act{nullptr, hidden_bf16}, out_ptrs, out_rows, count, batch,
                            in_cols, scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_dual_linear_f32(const uint8_t* wa, const float* sa, const uint8_t* wb,
                                              const float* sb, const float* hidden, float* out_a,
                                              float* out_b, int64_t batch, int64_t out_rows,
                                              int64_t in_cols, int64_t scale_cols) {
    if (!wa || !sa || !wb || !sb || !hidden || !out_a || !out_b) return plm::fail(-1, "null pointer");
    return dual_linear_impl(wa, sa, wb, sb, Act{hidden, nullptr}, out_a, out_b, batch, out_rows, in_cols,
                            scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_dual_linear_bf16x_f32(const uint8_t* wa, const float* sa, const uint8_t* wb,
                                                    const float* sb, const uint16_t* hidden_bf16, float* out_a,
                                                    float* out_b, int64_t batch, int64_t out_rows,
                                                    int64_t in_cols, int64_t scale_cols) {
    if (!wa || !sa || !wb || !sb || !hidden_bf16 || !out_a || !out_b) return plm::fail(-1, "null pointer");
    return dual_linear_impl(wa, sa, wb, sb, Act{nullptr, hidden_bf16}, out_a, out_b, batch, out_rows, in_cols,
                            scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_mlp_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                                      const uint8_t* up_weight, const float* up_scale_inv,
                                      const uint8_t* down_weight, const float* down_scale_inv,
                                      const float* hidden, float* out, int64_t batch,
                                      int64_t intermediate_rows, int64_t hidden_cols,
                                      int64_t gate_scale_cols, int64_t down_scale_cols) {
    if (!gate_weight || !gate_scale_inv || !up_weight || !up_scale_inv || !down_weight || !down_scale_inv ||
        !hidden || !out)
        return plm::fail(-1, "null pointer");
    return mlp_impl(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv,
                    Act{hidden, nullptr}, out, batch, intermediate_rows, hidden_cols, gate_scale_cols,
                    down_scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_mlp_bf16x_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                                            const uint8_t* up_weight, const float* up_scale_inv,
                                            const uint8_t* down_weight, const float* down_scale_inv,
                                            const uint16_t* hidden_bf16, float* out, int64_t batch,
                                            int64_t intermediate_rows, int64_t hidden_cols,
                                            int64_t gate_scale_cols, int64_t down_scale_cols) {
    if (!gate_weight || !gate_scale_inv || !up_weight || !up_scale_inv || !down_weight || !down_scale_inv ||
        !hidden_bf16 || !out)
        return plm::fail(-1, "null pointer");
    return mlp_impl(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight, down_scale_inv,
                    Act{nullptr, hidden_bf16}, out, batch, intermediate_rows, hidden_cols, gate_scale_cols,
                    down_scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_mlp_avx512_f32(const uint8_t* gate_weight, const float* gate_scale_inv,
                                             const uint8_t* up_weight, const float* up_scale_inv,
                                             const uint8_t* down_weight, const float* down_scale_inv,
                                             const float* hidden, float* out, int64_t batch,
                                             int64_t intermediate_rows, int64_t hidden_cols,
                                             int64_t gate_scale_cols, int64_t down_scale_cols) {
    return fp8_e4m3_block_mlp_f32(gate_weight, gate_scale_inv, up_weight, up_scale_inv, down_weight,
                                  down_scale_inv, hidden, out, batch, intermediate_rows, hidden_cols,
                                  gate_scale_cols, down_scale_cols);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_f32(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                                           const uint64_t* usp, const uint64_t* dp, const uint64_t* dsp,
                                           const float* hidden, float* out, int64_t expert_count,
                                           int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                                           int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !out) return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    hipStream_t st = plm::current_stream();
    float* act = static_cast<float*>(plm::workspace(static_cast<size_t>(expert_count * batch * inter) * sizeof(float)));
    if (act == nullptr) return -3;
    ExpertTables t(gp, gsp, up, usp, dp, dsp, expert_count);
    int code = gate_up_phase(t, expert_count, Act{hidden, nullptr}, act, batch, inter, hid, gsc, st);
    if (code != 0) return code;
    CombineProblem c;
    std::memset(&c, 0, sizeof(c));
    c.w = t.d.data();
    c.s = t.ds.data();
    c.ngroups = static_cast<int>(expert_count);
    c.act = act;
    c.per_group_out = true;
    c.out = out;
    c.batch = batch;
    c.rows = hid;
    c.K = inter;
    c.scale_cols = dsc;
    return run_combine(c, st);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_weighted_f32(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                                                    const uint64_t* usp, const uint64_t* dp, const uint64_t* dsp,
                                                    const float* hidden, const float* route_weights, float* out,
                                                    int64_t expert_count, int64_t batch, int64_t inter,
                                                    int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !route_weights || !out)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{hidden, nullptr}, route_weights, 1, 0, false, out,
                        expert_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_weighted_shared_f32(const uint64_t* gp, const uint64_t* gsp,
                                                           const uint64_t* up, const uint64_t* usp,
                                                           const uint64_t* dp, const uint64_t* dsp,
                                                           const float* hidden, const float* route_weights,
                                                           float* out, float* out_shared, int64_t expert_count,
                                                           int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                                                           int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !route_weights || !out || !out_shared)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    if (expert_count + 1 > kMaxGroups) return plm::fail(-2, "at most %d routed experts with a shared one", kMaxGroups - 1);
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{hidden, nullptr}, route_weights, 1, 0, false, out,
                        expert_count, batch, inter, hid, gsc, dsc, out_shared);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_weighted_bf16x_f32(const uint64_t* gp, const uint64_t* gsp,
                                                          const uint64_t* up, const uint64_t* usp,
                                                          const uint64_t* dp, const uint64_t* dsp,
                                                          const uint16_t* hidden_bf16, const float* route_weights,
                                                          float* out, int64_t expert_count, int64_t batch,
                                                          int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden_bf16 || !route_weights || !out)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{nullptr, hidden_bf16}, route_weights, 1, 0, false, out,
                        expert_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_weighted_shared_bf16x_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const uint16_t* hidden_bf16, const float* route_weights, float* out, float* out_shared,
    int64_t expert_count, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden_bf16 || !route_weights || !out || !out_shared)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    if (expert_count + 1 > kMaxGroups) return plm::fail(-2, "at most %d routed experts with a shared one", kMaxGroups - 1);
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{nullptr, hidden_bf16}, route_weights, 1, 0, false, out,
                        expert_count, batch, inter, hid, gsc, dsc, out_shared);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_weighted_avx512_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const float* hidden, const float* route_weights, float* out, int64_t expert_count,
    int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    return fp8_e4m3_block_mlp_many_weighted_f32(gp, gsp, up, usp, dp, dsp, hidden, route_weights, out,
                                                expert_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_row_weighted_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const float* hidden, const float* route_weights, float* out, int64_t expert_count,
    int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !route_weights || !out)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{hidden, nullptr}, route_weights, batch, 1, true, out,
                        expert_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_row_weighted_bf16x_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const uint16_t* hidden_bf16, const float* route_weights, float* out, int64_t expert_count,
    int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden_bf16 || !route_weights || !out)
        return plm::fail(-1, "null pointer");
    if (moe_dims_bad(expert_count, batch, inter, hid, gsc, dsc)) return plm::fail(-2, "bad dimensions");
    return weighted_moe(gp, gsp, up, usp, dp, dsp, Act{nullptr, hidden_bf16}, route_weights, batch, 1, true, out,
                        expert_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_pair_weighted_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const float* hidden, const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int64_t expert_count, int64_t pair_count, int64_t batch, int64_t inter,
    int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !pair_item_indices || !pair_row_indices ||
        !pair_weights || !out)
        return plm::fail(-1, "null pointer");
    return pair_weighted_impl(gp, gsp, up, usp, dp, dsp, Act{hidden, nullptr}, pair_item_indices, pair_row_indices,
                              pair_weights, out, expert_count, pair_count, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_pair_weighted_bf16x_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const uint16_t* hidden_bf16, const int64_t* pair_item_indices,
    const int64_t* pair_row_indices, const float* pair_weights, float* out, int64_t expert_count, int64_t pair_count,
    int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden_bf16 || !pair_item_indices || !pair_row_indices ||
        !pair_weights || !out)
        return plm::fail(-1, "null pointer");
    return pair_weighted_impl(gp, gsp, up, usp, dp, dsp, Act{nullptr, hidden_bf16}, pair_item_indices,
                              pair_row_indices, pair_weights, out, expert_count, pair_count, batch, inter, hid, gsc,
                              dsc);
}

// The pair-weighted MoE without the host read-back: pairs out of range are
// left out and counted into *bad_pairs (device memory).  No counterpart in
// the reference; for callers that must not wait on the stream (graph
// capture, the verifier batch).
PLM_EXPORT int fp8_e4m3_block_mlp_many_pair_weighted_nosync_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const float* hidden, const int64_t* pair_item_indices, const int64_t* pair_row_indices,
    const float* pair_weights, float* out, int* bad_pairs, int64_t expert_count, int64_t pair_count, int64_t batch,
    int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden || !pair_item_indices || !pair_row_indices ||
        !pair_weights || !out || !bad_pairs)
        return plm::fail(-1, "null pointer");
    return pair_weighted_impl(gp, gsp, up, usp, dp, dsp, Act{hidden, nullptr}, pair_item_indices, pair_row_indices,
                              pair_weights, out, expert_count, pair_count, batch, inter, hid, gsc, dsc, bad_pairs);
}

PLM_EXPORT int fp8_e4m3_block_mlp_many_pair_weighted_nosync_bf16x_f32(
    const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp, const uint64_t* dp,
    const uint64_t* dsp, const uint16_t* hidden_bf16, const int64_t* pair_item_indices,
    const int64_t* pair_row_indices, const float* pair_weights, float* out, int* bad_pairs, int64_t expert_count,
    int64_t pair_count, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !hidden_bf16 || !pair_item_indices || !pair_row_indices ||
        !pair_weights || !out || !bad_pairs)
        return plm::fail(-1, "null pointer");
    return pair_weighted_impl(gp, gsp, up, usp, dp, dsp, Act{nullptr, hidden_bf16}, pair_item_indices,
                              pair_row_indices, pair_weights, out, expert_count, pair_count, batch, inter, hid, gsc,
                              dsc, bad_pairs);
}

PLM_EXPORT int fp8_e4m3_block_moe_device_routed_f32(const uint64_t* expert_table, int64_t num_experts,
                                                    const int64_t* route_indices, const float* route_weights,
                                                    int64_t top_k, const uint64_t* shared_ptrs, const float* hidden,
                                                    float* out, float* out_shared, uint16_t* out_bf16,
                                                    int* rejected, int64_t batch, int64_t inter, int64_t hid,
                                                    int64_t gsc, int64_t dsc) {
    if (!expert_table || !route_indices || !route_weights || !hidden || !out || (shared_ptrs && !out_shared))
        return plm::fail(-1, "null pointer");
    return device_routed_impl(expert_table, num_experts, route_indices, route_weights, top_k, shared_ptrs,
                              Act{hidden, nullptr}, out, out_shared, out_bf16, rejected, batch, inter, hid, gsc, dsc);
}

PLM_EXPORT int fp8_e4m3_block_moe_device_routed_bf16x_f32(const uint64_t* expert_table, int64_t num_experts,
                                                          const int64_t* route_indices, const float* route_weights,
                                                          int64_t top_k, const uint64_t* shared_ptrs,
                                                          const uint16_t* hidden_bf16, float* out, float* out_shared,
                                                          uint16_t* out_bf16, int* rejected, int64_t batch,
                                                          int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!expert_table || !route_indices || !route_weights || !hidden_bf16 || !out || (shared_ptrs && !out_shared))
        return plm::fail(-1, "null pointer");
    return device_routed_impl(expert_table, num_experts, route_indices, route_weights, top_k, shared_ptrs,
                              Act{nullptr, hidden_bf16}, out, out_shared, out_bf16, rejected, batch, inter, hid, gsc,
                              dsc);
}

PLM_EXPORT int fp8_e4m3_block_moe_device_routed_bf16x_f32_noalloc(
    const uint64_t* expert_table, int64_t num_experts, const int64_t* route_indices, const float* route_weights,
    int64_t top_k, const uint64_t* shared_ptrs, const uint16_t* hidden_bf16, float* out, float* out_shared,
    uint16_t* out_bf16, int* rejected, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!expert_table || !route_indices || !route_weights || !hidden_bf16 || !out || (shared_ptrs && !out_shared))
        return plm::fail(-1, "null pointer");
    char* buf = nullptr;
    const int code = scratch_address(&buf);
    if (code != 0) return code;
    return device_routed_impl(expert_table, num_experts, route_indices, route_weights, top_k, shared_ptrs,
                              Act{nullptr, hidden_bf16}, out, out_shared, out_bf16, rejected, batch, inter, hid, gsc,
                              dsc, buf, kNoAllocScratchBytes);
}

PLM_EXPORT int fp8_e4m3_block_moe_from_logits_bf16x_f32(
    const float* router_logits, const float* router_bias, int64_t n_groups, int64_t topk_groups, int scoring,
    float route_scale, const uint64_t* expert_table, int64_t num_experts, int64_t top_k, const uint64_t* shared_ptrs,
    const uint16_t* hidden_bf16, float* out, float* out_shared, uint16_t* out_bf16, int64_t* out_indices,
    float* out_weights, int* rejected, int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!router_logits || !expert_table || !hidden_bf16 || !out || (shared_ptrs && !out_shared) ||
        ((out_indices == nullptr) != (out_weights == nullptr)))
        return plm::fail(-1, "null pointer");
    if (num_experts <= 0 || num_experts > 4096 || top_k <= 0 || top_k > num_experts || n_groups <= 0 ||
        n_groups > 64 || num_experts % n_groups != 0 || (scoring != 0 && scoring != 1))
        return plm::fail(-2, "bad routing dimensions");
    const RouteFromLogits route = {router_logits, router_bias, static_cast<int>(n_groups),
                                   static_cast<int>(topk_groups), scoring, route_scale};
    return device_routed_impl(expert_table, num_experts, out_indices, out_weights, top_k, shared_ptrs,
                              Act{nullptr, hidden_bf16}, out, out_shared, out_bf16, rejected, batch, inter, hid, gsc,
                              dsc, nullptr, 0, &route);
}

// Used by the DeepSeek session entry points (ds_session.hip).
int plm_weighted_moe_fp8(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up, const uint64_t* usp,
                         const uint64_t* dp, const uint64_t* dsp, const float* hidden, const float* route,
                         float* out, int64_t experts, int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                         int64_t dsc) {
    return fp8_e4m3_block_mlp_many_weighted_f32(gp, gsp, up, usp, dp, dsp, hidden, route, out, experts, batch,
                                                inter, hid, gsc, dsc);
}
