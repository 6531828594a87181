// FP8 e4m3 block-scaled GEMV family for gfx950: linear, dual linear, SwiGLU
// MLP and the (weighted) many-expert MoE of src/pcketlm/native/fp8_linear.cpp.
//
// Design.  The path is HBM-bound (2 flop per weight byte at one activation
// row), so every kernel streams each weight byte once per call, for all
// activation rows, with 16-byte nontemporal loads, and does the dot products
// on the matrix cores (v_mfma_f32_16x16x32_bf16; e4m3 -> bf16 is exact).
// Activation rows are MFMA columns and a column's result depends on that
// column alone, so a batched call returns, row for row, the bits of per-row
// calls (the reference's batch-reuse tests).  NaN weight bytes contribute 0
// (fp8_linear.cpp:31-33): a wave whose sums come out NaN runs its blocks
// again with NaN bytes zeroed.
//
// fp8_rows_kernel  : rows of one or more experts sharing the activations
//                    (linear, dual, gate/up phase with the SiLU epilogue, and
//                    several weights of different row counts in one grid);
//                    the activations are fp32 (split into bf16 hi + lo) or
//                    bf16 (the *_bf16x_f32 entry points); at one to four
//                    activation rows the lanes of B columns past the batch
//                    share the activation loads; for the device-routed MoE
//                    its first workgroup writes the plan of the router's
//                    choices.
// fp8_down_kernel  : rows whose K range is the concatenation of several
//                    experts' down matrices, each with its own activations
//                    (the SiLU intermediate as bf16 hi / lo planes) and route
//                    weight (down phase + routed combine); a last group can
//                    be split off into its own output (the shared expert
//                    beside the routed sum).
#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <vector>

#include "common.h"
#include "route.h"

// Loads of down-phase items (or lanes) that do not count read these zero
// bytes instead, so no load sits behind a branch: the compiler can then wait
// for each pipeline slot alone rather than for every load in flight.  The
// kernel gets the address as an argument (looked up per device), so the
// loads cannot be folded away as reads of a never-written array.
static __device__ __align__(256) unsigned char down_zero_page[256];

namespace {

constexpr int kMaxGroups = 64;  // experts per launch (pointer tables travel as kernel arguments)
constexpr int kMaxWaves = 8;
constexpr int kMaxM = 8;        // activation rows per launch; larger batches are split
constexpr int kMaxVar = 8;      // matrices of different row counts per many-linear launch

// Experts chosen on the device (the device-routed MoE).  The plan holds,
// for the sorted distinct experts of the router's [batch][top_k]
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
    int nblocks;          // 128-column blocks per row: ceil(K / 128)
    int m_total;
    int m0;
    int mc;               // activation rows of this launch (m0 .. m0 + mc - 1), at most kMaxM
    uint16_t* hhi;        // SiLU epilogue: the bf16 hi / lo planes of silu(gate) * up, element (g, m, row)
    uint16_t* hlo;        //   at ((g * m_total + m) * out_ld + row)
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
    int nw;  // waves per workgroup (the block size over 64)
    // Weights in 8-row tiles (fp8_e4m3_pack_tiles8): the byte of row r,
    // column c sits at ((r / 8) * nblocks + c / 128) * 1024 + (r % 8) * 128
    // + c % 128.  Only the weight addresses change.
    int tiled;
    // The plan made in the gate/up launch (the device-routed MoE, inplan =
    // 1): the grid's first workgroup writes the plan for the down phase from
    // the router's choices pidx / pwts [pbatch][ptop_k] and the device table
    // ptable [6][pexperts], and each device-chosen group finds its expert
    // from the choices itself instead of reading the plan.
    int inplan;
    int pbatch;
    int ptop_k;
    int64_t pexperts;
    const uint64_t* ptable;
    const int64_t* pidx;
    const float* pwts;
    MoePlan* pout;
    int* prejected;
};

// Byte offset of column offset off (a multiple of 16) from a weight row's
// base: off itself in a row-major row, and off plus 896 bytes per 128-column
// block in an 8-row tile row (each block of a tile row is 1 KB from the last).
__device__ __forceinline__ int64_t tile_col(int64_t off, int tiled) { return off + (tiled ? (off >> 7) * 896 : 0); }

struct CombineArgs {
    const uint8_t* w[kMaxGroups];
    const float* s[kMaxGroups];
    const uint16_t* act_hi;  // activations of group g, bf16 hi / lo planes of the SiLU intermediate:
    const uint16_t* act_lo;  //   element ((g_base+g)*m_total + m) * K + col
    const float* route;   // route of (g, m): route[(g_base+g)*route_sg + m*route_sm], or null (= 1)
    float* out;
    int64_t rows;
    int64_t K;
    int64_t scale_cols;
    int64_t route_sg;
    int64_t route_sm;
    int ngroups;
    int g_base;
    int nbe;              // 128-column blocks per group segment
    int tiles_per_group;  // per_group_out only
    int per_group_out;    // 1: out[(g_base+g)*m_total + m][row]; 0: out[m][row] summed over groups
    int split_last;       // (summed mode) the last group is not summed: its own tiles write it, with
                          // route 1, to out_last[m][row]
    float* out_last;
    int accumulate;       // add to out instead of storing
    int zero_skip;        // skip (g, m) whose route is exactly 0
    int m_total;
    int m0;
    int mc;               // activation rows of this launch
    const MoePlan* plan;  // as in RowsArgs (tab rows 4-5 for the down matrices)
    int ndev;
    int fused;            // the split-off last group computed by the routed workgroups (fp8_down_kernel FUSED)
    uint16_t* out_bf16;   // summed mode: bf16(bf16(out) + bf16(out_last)) (no split-off group: bf16(out)), or null
    int rows_per_wg;      // fp8_down_kernel: output rows per workgroup (at most kDownMaxRows)
    const unsigned char* zero;  // fp8_down_kernel: 256 zero bytes in device memory
};

static_assert(kMaxGroups == 64, "the plan maps one lane of the first wave to each group");
struct PlanShared {
    int64_t key[64];
    float kw[64];
    int first[64];
    int64_t sel[kMaxGroups];
};

// The plan of the router's n = batch * top_k choices (n <= 64) as
// run_fp8_moe builds it on the host (fp8_source.py:1600, 1653-1716): the
// distinct in-range experts in ascending order, their addresses from the
// device table [6][num_experts], and the route matrix [group][batch] (a
// row's weight for the expert, 0 when the row did not choose it; a repeated
// index within a row keeps its first weight).  An index outside
// [0, num_experts) is left out; an expert whose weight addresses are not
// 16-byte aligned (scales: 4) keeps its group but gets null addresses, so it
// contributes nothing.  Both are counted in *rejected.  Run by a whole
// workgroup (every thread calls it: it synchronises the workgroup); the
// first wave does the work.
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

// The expert of device-chosen group g as plan_from_choices numbers the
// groups (the distinct in-range choices of the n = batch * top_k, in
// ascending order) and its six table addresses, all null when any of them is
// misaligned; returns the number of groups.  One wave does it alone, in two
// memory round trips (the choices, then the expert's table entries).
__device__ __forceinline__ int group_expert(const uint64_t* __restrict__ table, int64_t num_experts,
                                            const int64_t* __restrict__ idx, int n, int g, int lane,
                                            uint64_t (&ad)[kPlanRoles]) {
    const int64_t v = lane < n ? idx[lane] : -1;
    const int e = v >= 0 && v < num_experts ? static_cast<int>(v) : -1;
    bool first = e >= 0;  // no earlier choice names the same expert
    for (int i = 0; i < n; ++i) first = first && !(i < lane && __builtin_amdgcn_readlane(e, i) == e);
    const uint64_t fm = __ballot(first);
    const int count = __popcll(fm);
    if (g >= count) return count;
    int rank = 0;
    for (int i = 0; i < n; ++i) rank += static_cast<int>((fm >> i) & 1) & (__builtin_amdgcn_readlane(e, i) < e);
    const int eg = __builtin_amdgcn_readlane(e, __builtin_ctzll(__ballot(first && rank == g)));
#pragma unroll
    for (int r = 0; r < kPlanRoles; ++r) ad[r] = table[static_cast<int64_t>(r) * num_experts + eg];
    bool aligned = true;
#pragma unroll
    for (int r = 0; r < kPlanRoles; ++r) aligned = aligned && (ad[r] & ((r & 1) ? 3u : 15u)) == 0;
#pragma unroll
    for (int r = 0; r < kPlanRoles; ++r) {
        const uint64_t v = aligned ? ad[r] : 0;
        ad[r] = (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v >> 32)))) << 32) |
                static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
    }
    return count;
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
__device__ __forceinline__ void route_plan_body(const float* __restrict__ logits, const float* __restrict__ bias,
                                                int experts, int batch, int top_k, int n_groups, int topk_groups,
                                                int scoring, float route_scale, const uint64_t* __restrict__ table,
                                                int64_t* idx_out, float* w_out, MoePlan* __restrict__ plan,
                                                int* __restrict__ rejected) {
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
            // unconditional loads (rows past the table read its last entry;
            // the router never picks them), first used after the routing
#pragma unroll
            for (int r = 0; r < kPlanRoles; ++r)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    tab[r][j] = table[static_cast<int64_t>(r) * experts + min(4 * lane + j, experts - 1)];
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

template <int J>
__global__ __launch_bounds__(512) void moe_route_plan_kernel(const float* __restrict__ logits,
                                                            const float* __restrict__ bias, int experts, int batch,
                                                            int top_k, int n_groups, int topk_groups, int scoring,
                                                            float route_scale, const uint64_t* __restrict__ table,
                                                            int64_t* idx_out, float* w_out,
                                                            MoePlan* __restrict__ plan, int* __restrict__ rejected) {
    route_plan_body<J>(logits, bias, experts, batch, top_k, n_groups, topk_groups, scoring, route_scale, table,
                       idx_out, w_out, plan, rejected);
}

// ------------------------------------------------------------------ matrix-core tiles
//
// A tile is 8 weight rows by one 128-column block (one block of the scale
// grid).  The 16 rows of the A operand of v_mfma_f32_16x16x32_bf16 are the
// pairs (weight row r, half h) = (i & 7, i >> 3): lane l (i = l & 15,
// quarter q = l >> 4) loads the 16 bytes at columns 64h + 16q of row r, so
// one load instruction reads 8 whole 128-byte lines.  The 16 columns of the
// B operand are the pairs (activation row m, half h') = (n & 7, n >> 3) and
// hold the same columns of activation row m, so D[(r, h)][(m, h')] is the
// dot of weight row r with activation row m over half h of the block when
// h == h' (the other half of D is not used).  The lane's 16 bytes are two
// MFMAs' worth (8 bf16 each); e4m3 -> bf16 is exact.  Each block's D is
// scaled into the accumulators, acc = fma(D, scale, acc), and the two halves
// are added after the last block, acc(h = 0) + acc(h = 1).
//
// Activation rows are MFMA columns: a column's result depends only on that
// column's inputs, so an M-row call returns, row for row, the bits of M
// one-row calls.  bf16 activations are one B operand; fp32 activations are
// split into hi (the upper 16 bits) + lo (the remainder rounded to bf16),
// two more MFMAs, within 2^-17 relative of the fp32 value.
//
// NaN weight bytes count as 0 (fp8_linear.cpp:31-33).  The hot loop decodes
// them as NaN; a wave whose accumulators come out NaN runs its blocks again
// with NaN bytes zeroed and infinite or NaN activations split exactly (hi =
// the value, lo = 0).  Rows and activations without such values give the
// same bits in both passes.

typedef __bf16 plm_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 plm_bf16x2 __attribute__((ext_vector_type(2)));
typedef float plm_f32x4 __attribute__((ext_vector_type(4)));

// Weight bytes are read once per call: nontemporal loads keep them from
// displacing the activations and scales in the caches.
__device__ __forceinline__ plm_u32x4 wload16(const void* p) {
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) plm_u32x4*)(p));
}

__device__ __forceinline__ plm_u32x4 xload16(const void* p) {
    return *(const __attribute__((address_space(1))) plm_u32x4*)(p);
}

template <bool HI>
__device__ __forceinline__ uint32_t e4m3_pair_to_bf16(uint32_t v) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, 1.0f, HI));
}

// 16 e4m3 bytes -> the two A operands (bytes 0-7, 8-15)
__device__ __forceinline__ void weights_to_bf16(const plm_u32x4 q, plm_bf16x8& a0, plm_bf16x8& a1) {
    const plm_u32x4 t0 = {e4m3_pair_to_bf16<false>(q.x), e4m3_pair_to_bf16<true>(q.x),
                          e4m3_pair_to_bf16<false>(q.y), e4m3_pair_to_bf16<true>(q.y)};
    const plm_u32x4 t1 = {e4m3_pair_to_bf16<false>(q.z), e4m3_pair_to_bf16<true>(q.z),
                          e4m3_pair_to_bf16<false>(q.w), e4m3_pair_to_bf16<true>(q.w)};
    a0 = __builtin_bit_cast(plm_bf16x8, t0);
    a1 = __builtin_bit_cast(plm_bf16x8, t1);
}

// NaN bytes (0x7F, 0xFF) -> 0
__device__ __forceinline__ plm_u32x4 zero_nan_bytes(plm_u32x4 q) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t w = q[k];
        const uint32_t nan = ((w & 0x7F7F7F7Fu) + 0x01010101u) & 0x80808080u;  // 0x80 where the low 7 bits are all 1
        q[k] = w & ~((nan >> 7) * 0xFFu);
    }
    return q;
}

// hi / lo bf16 halves of one fp32 value.  EXACT: infinities and NaNs go to hi
// whole (a quiet NaN for every NaN) with lo = 0.
template <bool EXACT>
__device__ __forceinline__ void split_f32(uint32_t x, uint32_t& hi, uint32_t& lo) {
    hi = x >> 16;
    const float rem = __uint_as_float(x) - __uint_as_float(x & 0xFFFF0000u);
    lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(rem));
    if constexpr (EXACT) {
        if ((x & 0x7F800000u) == 0x7F800000u) {
            hi = (x & 0x007FFFFFu) != 0 ? 0x7FC0u : hi;
            lo = 0;
        }
    }
}

// 8 fp32 activations (two loads) -> hi and lo B operands
template <bool EXACT>
__device__ __forceinline__ void split8(const plm_u32x4 v0, const plm_u32x4 v1, plm_bf16x8& hi, plm_bf16x8& lo) {
    const uint32_t x[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    plm_u32x4 h, l;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        if constexpr (EXACT) {
            uint32_t h0, l0, h1, l1;
            split_f32<true>(x[2 * p], h0, l0);
            split_f32<true>(x[2 * p + 1], h1, l1);
            h[p] = h0 | (h1 << 16);
            l[p] = l0 | (l1 << 16);
        } else {
            h[p] = __builtin_amdgcn_perm(x[2 * p + 1], x[2 * p], 0x07060302u);
            const float r0 = __uint_as_float(x[2 * p]) - __uint_as_float(x[2 * p] & 0xFFFF0000u);
            const float r1 = __uint_as_float(x[2 * p + 1]) - __uint_as_float(x[2 * p + 1] & 0xFFFF0000u);
            const plm_float2 rr = {r0, r1};
            l[p] = __builtin_bit_cast(uint32_t, __builtin_convertvector(rr, plm_bf16x2));
        }
    }
    hi = __builtin_bit_cast(plm_bf16x8, h);
    lo = __builtin_bit_cast(plm_bf16x8, l);
}

__device__ __forceinline__ plm_f32x4 mfma_bf16(plm_bf16x8 a, plm_bf16x8 b, plm_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// The activations of one block for the lane's B column: two bf16 loads, or
// four fp32 loads (split into hi and lo later).
template <bool XB>
struct XPiece {
    plm_u32x4 v[XB ? 2 : 4];
};

template <bool XB>
__device__ __forceinline__ XPiece<XB> load_xpiece(const void* p, bool live) {
    XPiece<XB> r;
    const char* c = static_cast<const char*>(p);
#pragma unroll
    for (int k = 0; k < (XB ? 2 : 4); ++k) r.v[k] = live ? xload16(c + 16 * k) : plm_u32x4{0, 0, 0, 0};
    return r;
}

// D of one tile and block: the A operands from the weights q against the
// activation piece x.
template <bool XB, bool SAN>
struct BOperands {
    plm_bf16x8 h0, h1, l0, l1;
    __device__ __forceinline__ explicit BOperands(const XPiece<XB>& x) {
        if constexpr (XB) {
            h0 = __builtin_bit_cast(plm_bf16x8, x.v[0]);
            h1 = __builtin_bit_cast(plm_bf16x8, x.v[1]);
        } else {
            split8<SAN>(x.v[0], x.v[1], h0, l0);
            split8<SAN>(x.v[2], x.v[3], h1, l1);
        }
    }
};

template <bool XB, bool SAN>
__device__ __forceinline__ plm_f32x4 tile_block(plm_u32x4 q, const BOperands<XB, SAN>& b) {
    plm_bf16x8 a0, a1;
    weights_to_bf16(SAN ? zero_nan_bytes(q) : q, a0, a1);
    plm_f32x4 d = mfma_bf16(a0, b.h0, plm_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
    d = mfma_bf16(a1, b.h1, d);
    if constexpr (!XB) {
        d = mfma_bf16(a0, b.l0, d);
        d = mfma_bf16(a1, b.l1, d);
    }
    return d;
}

template <int NT>
__device__ __forceinline__ bool any_nan(const plm_f32x4 (&acc)[NT]) {
    bool bad = false;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) bad = bad || acc[t][j] != acc[t][j];
    return __any(bad);
}

// Adds the two halves and leaves tile t's sums of this wave in LDS:
// red[(slot * NT + t) * 64 + r * 8 + m] for weight row r, activation row m.
template <int NT>
__device__ __forceinline__ void halves_to_lds(const plm_f32x4 (&acc)[NT], float* red, int slot, int lane) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = acc[t][j] + __shfl(acc[t][j], (lane + 40) & 63);
            if (lane < 24 && (lane & 15) < 8) red[(slot * NT + t) * 64 + (4 * (lane >> 4) + j) * 8 + (lane & 7)] = v;
        }
}

// The SiLU intermediate silu(gate) * up as the down phase reads it: bf16
// hi / lo planes (exact for infinities and NaNs).
__device__ __forceinline__ void store_hplanes(uint16_t* hi, uint16_t* lo, int64_t o, float v) {
    uint32_t h, l;
    split_f32<true>(__float_as_uint(v), h, l);
    hi[o] = static_cast<uint16_t>(h);
    lo[o] = static_cast<uint16_t>(l);
}

__device__ __forceinline__ float lane_value(float v, int k) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), k));
}

// Runs nk steps through P register slots, pipelined: P steps are in
// flight and step k + P is issued into the slot step k leaves; the steps
// beyond a multiple of P run first, unpipelined.
template <int P, class Issue, class Compute>
__device__ __forceinline__ void run_pipelined(int nk, Issue& issue, Compute& compute) {
    const int r = nk % P;
    for (int k = 0; k < r; ++k) {
        issue(0, k);
        compute(0, k);
    }
    if (nk > r) {
#pragma unroll
        for (int u = 0; u < P; ++u) issue(u, r + u);
        for (int k0 = r; k0 + P < nk; k0 += P) {
#pragma unroll
            for (int u = 0; u < P; ++u) {
                compute(u, k0 + u);
                issue(u, k0 + u + P);
            }
        }
#pragma unroll
        for (int u = 0; u < P; ++u) compute(u, nk - P + u);
    }
}

// The burst schedule of a rows-kernel wave (the MoE's gate/up launches):
// the loads of U blocks b = b0, b0 + nw, ... are issued together, then the
// U blocks are consumed.  Activations are loaded by the lanes of live rows
// only and scales per block.
// v of lane K of the lane's quad (lanes 4j .. 4j + 3).
template <int K>
__device__ __forceinline__ plm_u32x4 quad_part(plm_u32x4 v) {
    plm_u32x4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        r[c] = static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v[c]), K * 0x55, 0xF, 0xF, false));
    return r;
}

// One activation row (X1, the linear family's loop, where every lane reads
// a piece: lanes of B columns past the batch read row 0's): the lanes of a
// quad (activation rows m = 0-3 of one B column half and quarter) hold the
// same piece, so each loads one 16-byte part of it and the parts are
// exchanged across the quad, one load instruction per block instead of two
// (bf16) or four (fp32).  o 7168x16384 at one row: 26.2 -> 23.0 us (bf16),
// 36.2 -> 28.9 us (fp32).  The gate/up burst loop loads on the live lanes
// only and gains nothing from it.
template <bool XB>
__device__ __forceinline__ plm_u32x4 load_xpart(const char* piece, int lane) {
    return xload16(piece + 16 * ((lane & 3) % (XB ? 2 : 4)));
}
// Two to four activation rows (XS == 2): the lanes of B columns of rows
// 4-7 are past the batch, so lane m + 4 (the next quad of its row of 16)
// loads the second half of row m's piece and the halves are swapped between
// the two lanes with DPP row shifts: one load instruction per block instead
// of two (bf16), two instead of four (fp32).
template <bool XB>
__device__ __forceinline__ const char* pair_half(const char* piece, int lane) {
    return piece + ((lane >> 2) & 1) * (XB ? 16 : 32);
}
__device__ __forceinline__ plm_u32x4 pair_swap(plm_u32x4 v, bool upper) {
    plm_u32x4 r;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int from_up = __builtin_amdgcn_mov_dpp(static_cast<int>(v[c]), 0x104, 0xF, 0xF, false);  // row_shl:4
        const int from_lo = __builtin_amdgcn_mov_dpp(static_cast<int>(v[c]), 0x114, 0xF, 0xF, false);  // row_shr:4
        r[c] = static_cast<uint32_t>(upper ? from_lo : from_up);
    }
    return r;
}
template <bool XB>
__device__ __forceinline__ XPiece<XB> pair_piece(const XPiece<XB>& own, int lane) {
    const bool upper = ((lane >> 2) & 1) != 0;  // holds the second half
    XPiece<XB> x;
    if constexpr (XB) {
        const plm_u32x4 other = pair_swap(own.v[0], upper);
        x.v[0] = upper ? other : own.v[0];
        x.v[1] = upper ? own.v[0] : other;
    } else {
        const plm_u32x4 o0 = pair_swap(own.v[0], upper), o1 = pair_swap(own.v[1], upper);
        x.v[0] = upper ? o0 : own.v[0];
        x.v[1] = upper ? o1 : own.v[1];
        x.v[2] = upper ? own.v[0] : o0;
        x.v[3] = upper ? own.v[1] : o1;
    }
    return x;
}

template <bool XB>
__device__ __forceinline__ XPiece<XB> quad_piece(plm_u32x4 part) {
    XPiece<XB> x;
    x.v[0] = quad_part<0>(part);
    x.v[1] = quad_part<1>(part);
    if constexpr (!XB) {
        x.v[2] = quad_part<2>(part);
        x.v[3] = quad_part<3>(part);
    }
    return x;
}

template <int TT, int U, int NWT, bool XB, bool SAN>
__device__ __forceinline__ void rows_pass_burst(const RowsArgs& a, const uint8_t* const (&wrow)[NWT * TT],
                                                const float* const (&sp)[NWT], const char* xrow, bool xlive,
                                                int64_t lane_col, int wave, int nw, plm_f32x4 (&acc)[NWT * TT]) {
    constexpr int NT = NWT * TT;
    constexpr int XE = XB ? 2 : 4;  // bytes per activation
    const int64_t nb = a.nblocks;
    for (int64_t b0 = wave; b0 < nb; b0 += static_cast<int64_t>(U) * nw) {
        plm_u32x4 q[U][NT];
        XPiece<XB> x[U];
        float sc[U][NWT];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t b = b0 + static_cast<int64_t>(u) * nw;
            const int64_t off = b * 128 + lane_col;
            const bool in = b < nb && off < a.K;
            const int64_t woff = tile_col(off, a.tiled);
#pragma unroll
            for (int t = 0; t < NT; ++t) q[u][t] = in ? wload16(wrow[t] + woff) : plm_u32x4{0, 0, 0, 0};
            x[u] = load_xpiece<XB>(xrow + off * XE, xlive && in);
#pragma unroll
            for (int n = 0; n < NWT; ++n) sc[u][n] = b < nb ? plm_gload_f32(sp[n] + b) : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const BOperands<XB, SAN> bo(x[u]);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const plm_f32x4 d = tile_block<XB, SAN>(q[u][t], bo);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(d[j], sc[u][t / TT], acc[t][j]);
            }
        }
    }
}

// One pass of a rows-kernel wave over its blocks b = wave + k nw, k = 0,
// 1, ...  Software-pipelined: P blocks are in flight, and block k + P is
// issued into the slot block k leaves.  No load sits behind a branch (a
// conditional load makes the compiler wait for every outstanding load
// before the next use): loads past the end of a row read its last 16
// bytes and are masked when used, activation rows past the batch read row
// 0 into B columns whose results are dropped, and the blocks beyond a
// multiple of P run first, unpipelined.  The wave's scales come first, one
// load for up to 64 blocks (lane k holds block k's), read with v_readlane.
// XS: how the activation pieces are loaded: 0 every lane its own, 1 one
// activation row (quad-shared parts), 2 two to four rows (pair-shared halves).
template <int TT, int P, int NWT, bool XB, bool SAN, int XS>
__device__ __forceinline__ void rows_pass(const RowsArgs& a, const uint8_t* const (&wrow)[NWT * TT],
                                          const float* const (&sp)[NWT], const char* xrow, int64_t lane_col,
                                          int wave, int nw, int lane, plm_f32x4 (&acc)[NWT * TT]) {
    constexpr int NT = NWT * TT;
    constexpr int XE = XB ? 2 : 4;  // bytes per activation
    const int64_t K = a.K;
    const bool ragged = (K & 127) != 0;
    const int64_t nb = a.nblocks;
    const int nk_all = wave < nb ? static_cast<int>((nb - 1 - wave) / nw) + 1 : 0;
    for (int kb = 0; kb < nk_all; kb += 64) {
        const int nk = min(nk_all - kb, 64);
        float sv[NWT];
        const int64_t sblk = wave + static_cast<int64_t>(kb + min(lane, nk - 1)) * nw;
#pragma unroll
        for (int n = 0; n < NWT; ++n) sv[n] = plm_gload_f32(sp[n] + sblk);
        plm_u32x4 q[P][NT];
        XPiece<XB> x[P];
        auto issue = [&](int slot, int k) {
            const int64_t off = min((wave + static_cast<int64_t>(kb + k) * nw) * 128 + lane_col, K - 16);
#pragma unroll
            for (int t = 0; t < NT; ++t) q[slot][t] = wload16(wrow[t] + tile_col(off, a.tiled));
            if constexpr (XS == 1) {
                x[slot].v[0] = load_xpart<XB>(xrow + off * XE, lane);
            } else if constexpr (XS == 2) {
                const char* h = pair_half<XB>(xrow + off * XE, lane);
                x[slot].v[0] = xload16(h);
                if constexpr (!XB) x[slot].v[1] = xload16(h + 16);
            } else {
                x[slot] = load_xpiece<XB>(xrow + off * XE, true);
            }
        };
        auto compute = [&](int slot, int k) {
            float sc[NWT];
#pragma unroll
            for (int n = 0; n < NWT; ++n) sc[n] = lane_value(sv[n], k);
            XPiece<XB> xv;
            if constexpr (XS == 1) {
                xv = quad_piece<XB>(x[slot].v[0]);
            } else if constexpr (XS == 2) {
                xv = pair_piece<XB>(x[slot], lane);
            } else {
                xv = x[slot];
            }
            plm_u32x4 qv[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) qv[t] = q[slot][t];
            if (ragged) {
                // the row's last block: columns past K add nothing
                const bool in = (wave + static_cast<int64_t>(kb + k) * nw) * 128 + lane_col < K;
#pragma unroll
                for (int t = 0; t < NT; ++t) qv[t] = in ? qv[t] : plm_u32x4{0, 0, 0, 0};
#pragma unroll
                for (int i = 0; i < (XB ? 2 : 4); ++i) xv.v[i] = in ? xv.v[i] : plm_u32x4{0, 0, 0, 0};
            }
            const BOperands<XB, SAN> bo(xv);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const plm_f32x4 d = tile_block<XB, SAN>(qv[t], bo);
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[t][j] = fmaf(d[j], sc[t / TT], acc[t][j]);
            }
        };
        run_pipelined<P>(nk, issue, compute);
    }
}

// Makes uniform values opaque to the compiler (touches no memory): the
// loads that produce them are issued together where they are pinned, one
// round trip, where a branch on each loaded value would cost one each.
__device__ __forceinline__ void pin_one(int& v) { asm("" : "+s"(v)); }
__device__ __forceinline__ void pin_one(int64_t& v) { asm("" : "+s"(v)); }
template <class T>
__device__ __forceinline__ void pin_one(T*& p) {
    uint64_t v = reinterpret_cast<uint64_t>(p);
    asm("" : "+s"(v));
    p = reinterpret_cast<T*>(v);
}
template <class... T>
__device__ __forceinline__ void pin_scalar(T&... v) {
    (pin_one(v), ...);
}

// Rows of one or more weights sharing the activations (linear, dual, the
// gate/up phase with its SiLU epilogue, weights of different row counts in
// one grid).  A workgroup owns TT tiles (8 TT rows) of each of its NWT
// weights; its nw waves split the K blocks (block b on wave b % nw), and nw
// depends only on K.  TT and U (blocks in flight per wave) change the grid
// and the schedule, never a row's arithmetic.
template <int TT, int U, bool BURST, int NWT, bool SILU, bool XB, bool INPLAN, int XS>
__device__ __forceinline__ void rows_tile(const RowsArgs& a, const int block) {
    static_assert(!INPLAN || (NWT == 2 && SILU), "the in-launch plan is the MoE gate/up phase's");
    static_assert(XS == 0 || !BURST, "the shared activation loads are the pipelined loop's");
    constexpr int NT = NWT * TT;
    __shared__ float red[kMaxWaves * NT * 64];
    // the arguments of the prologue and of the loop, read at once
    int nw = a.nw, tpg = a.tiles_per_group, nvar = a.nvar, mc = a.mc, m0 = a.m0, nb = a.nblocks;
    int tiled = a.tiled;
    int64_t rows = a.rows, K = a.K, scale_cols = a.scale_cols, x_stride = a.x_stride;
    const char* xbase = XB ? reinterpret_cast<const char*>(a.xb) : reinterpret_cast<const char*>(a.x);
    const uint8_t* w0[NWT];
    const float* s0[NWT];
#pragma unroll
    for (int i = 0; i < NWT; ++i) {
        w0[i] = a.w[i][0];
        s0[i] = a.s[i][0];
        pin_scalar(w0[i], s0[i]);
    }
    pin_scalar(nw, tpg, nvar, mc, m0, nb, tiled, rows, K, scale_cols, x_stride, xbase);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    // In-launch plan: the first workgroup writes the plan, after a pass
    // through the body as a tile with no weights (the plan's stores come
    // after every weight and scale load in program order, so the compiler
    // keeps those loads scalar where they are uniform).
    int tile = block;
    bool writer = false;
    if constexpr (INPLAN) {
        writer = block == 0;
        tile = max(block - 1, 0);
    }
    int g;
    int64_t row0;
    if (nvar > 0) {
        g = 0;
        for (int i = 1; i < a.nvar; ++i)
            if (tile >= a.vtile[i]) g = i;
        row0 = static_cast<int64_t>(tile - a.vtile[g]) * 8 * TT;
        rows = a.vrows[g];
    } else {
        g = tile / tpg;
        row0 = static_cast<int64_t>(tile - g * tpg) * 8 * TT;
    }

    const uint8_t* W[NWT];
    const float* S[NWT];
    int ga = g;  // argument slot
    if constexpr (NWT == 2 && SILU) {
        // (device-chosen groups exist only for the gate/up phase of the MoE)
        if (writer) {
#pragma unroll
            for (int i = 0; i < NWT; ++i) {
                W[i] = nullptr;
                S[i] = nullptr;
            }
        } else if (g < a.ndev) {
            if constexpr (INPLAN) {
                uint64_t ad[kPlanRoles];
                if (g >= group_expert(a.ptable, a.pexperts, a.pidx, a.pbatch * a.ptop_k, g, lane, ad)) return;
#pragma unroll
                for (int i = 0; i < NWT; ++i) {
                    W[i] = reinterpret_cast<const uint8_t*>(ad[2 * i]);
                    S[i] = reinterpret_cast<const float*>(ad[2 * i + 1]);
                }
            } else {
                if (g >= a.plan->count) return;  // the router chose fewer experts (uniform: before any barrier)
#pragma unroll
                for (int i = 0; i < NWT; ++i) {
                    W[i] = reinterpret_cast<const uint8_t*>(a.plan->tab[2 * i][g]);
                    S[i] = reinterpret_cast<const float*>(a.plan->tab[2 * i + 1][g]);
                }
            }
        }
        ga = writer ? -1 : g - a.ndev;
    }
    if (ga == 0) {
        // the first argument slot came with the other arguments
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            W[i] = w0[i];
            S[i] = s0[i];
        }
    } else if (ga > 0) {
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            W[i] = a.w[i][ga];
            S[i] = a.s[i][ga];
        }
    }
    bool live = true;
#pragma unroll
    for (int i = 0; i < NWT; ++i) live = live && W[i] != nullptr && S[i] != nullptr;

    const int li = lane & 15;
    const int64_t lane_col = 64 * (li >> 3) + 16 * (lane >> 4);
    const int xm = li & 7;  // activation row of this lane's B column
    const bool xlive = xm < mc;
    plm_f32x4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = plm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    if (live) {
        const uint8_t* wrow[NT];
        const float* sp[NWT];
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            sp[i] = S[i] + (row0 >> 7) * scale_cols;
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                // rows past the end read the last row; their results are dropped
                const int64_t r = min(row0 + 8 * t + (li & 7), rows - 1);
                wrow[i * TT + t] = tiled ? W[i] + ((r >> 3) * nb * 1024 + (r & 7) * 128) : W[i] + r * K;
            }
        }
        // XS == 2: lane m + 4 reads row m (rows 4-7 are past the batch)
        const int xr = XS == 2 ? (xm & 3) : xm;
        const int64_t xo = static_cast<int64_t>(m0 + (xr < mc ? xr : 0)) * x_stride;
        const char* xrow = xbase + xo * (XB ? 2 : 4);
        auto pass = [&](auto san) {
            constexpr bool SAN = decltype(san)::value;
            if constexpr (BURST)
                rows_pass_burst<TT, U, NWT, XB, SAN>(a, wrow, sp, xrow, xlive, lane_col, wave, nw, acc);
            else
                rows_pass<TT, U, NWT, XB, SAN, XS>(a, wrow, sp, xrow, lane_col, wave, nw, lane, acc);
        };
        pass(std::false_type{});
        if (any_nan(acc)) {
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[t] = plm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            pass(std::true_type{});
        }
    }
    halves_to_lds(acc, red, wave, lane);
    __syncthreads();

    for (int t = threadIdx.x; t < TT * 64; t += nw * 64) {
        const int tt = t >> 6, r = (t >> 3) & 7, m = t & 7;
        const int64_t row = row0 + 8 * tt + r;
        if (m >= a.mc || row >= rows || writer) continue;
        float v[NWT];
#pragma unroll
        for (int i = 0; i < NWT; ++i) {
            float s = 0.0f;
            for (int w = 0; w < nw; ++w) s += red[(w * NT + i * TT + tt) * 64 + r * 8 + m];
            v[i] = s;
        }
        const int64_t o = (static_cast<int64_t>(g) * a.m_total + a.m0 + m) * a.out_ld + row;
        if constexpr (SILU) {
            store_hplanes(a.hhi, a.hlo, o, plm_silu_mul(v[0], v[1]));
        } else {
            if (a.nvar > 0) {
                a.vout[g][static_cast<int64_t>(a.m0 + m) * rows + row] = v[0];
                continue;
            }
#pragma unroll
            for (int i = 0; i < NWT; ++i) a.out[i][o] = v[i];
        }
    }
    if constexpr (INPLAN) {
        if (writer) {
            __shared__ PlanShared ps;
            plan_from_choices(a.ptable, a.pexperts, a.pidx, a.pwts, a.pbatch, a.ptop_k, a.pout, a.prejected, ps);
        }
    }
}

template <int TT, int U, bool BURST, int NWT, bool SILU, bool XB, bool INPLAN = false, int XS = 0>
__global__ __launch_bounds__(512) void fp8_rows_kernel(const RowsArgs a) {
    rows_tile<TT, U, BURST, NWT, SILU, XB, INPLAN, XS>(a, static_cast<int>(blockIdx.x));
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

// What every item of a group needs (several activation rows: staged in LDS
// by the whole workgroup before its waves start): the down matrix, its
// scales and the route weight of each activation row.
struct GroupInfo {
    const uint8_t* w;
    const float* s;
    float rw[kMaxM];
};

// ------------------------------------------------------------------ down phase, one workgroup per CU
//
// fp8_down_kernel, laid out for the 256 compute units of the part:
//   * a workgroup of up to 16 waves owns rows_per_wg output rows (28 at
//     7168 rows: 256 workgroups, each streaming the same bytes) in up to 4
//     tiles of 8 rows.  Tiles start at multiples of 8 (the first and last
//     may be partial: rows outside the range are read again from its edge
//     and dropped), so a tile never crosses a 128-row scale block and its
//     scale is the same for the whole wave;
//   * items (group, block) go to waves round robin, nw = min(16, items), and
//     the wave sums are added in wave order: a row's arithmetic depends on
//     the items alone, never on the batch, the row range or the grid;
//   * each wave keeps P items in flight (a ring of P register slots; every
//     load is unconditional, slots past the wave's last item read a zero
//     page), so the compiler waits for one slot at a time;
//   * FUSED: the split-off last group (the shared expert) is computed by the
//     same workgroup, its items on the last waves when it has fewer items
//     than waves (the wave sums then equal those of a launch of that group
//     alone), and its first item is loaded before the plan of a
//     device-routed call is known.
// STAGE (one activation row): every wave reads the groups' addresses and
// route weights itself (lane g holds group g's) and copies the activations of
// its own items into its own LDS region, so no workgroup barrier stands
// before the weight stream.  Otherwise the workgroup stages the groups in
// LDS behind one barrier and each item also loads its activation pieces.
constexpr int kDownWaves = 16;
constexpr int kDownMaxRows = 32;
constexpr int kDownItemBytes = 512;    // one item's activations at one row: hi and lo planes of 128 columns
constexpr int kDownStageItems = 12;    // STAGE: items per wave at most (6 KB of LDS per wave)
constexpr int kDownStageLoads = kDownStageItems / 2;  // a wave load (1 KB) carries two items

template <class T>
__device__ __forceinline__ T* lane_ptr(T* p, int lane) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), lane);
    const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(v >> 32), lane);
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

// The address as a value the compiler cannot see through, so a load from
// "real or zero page" stays one unconditional load (it would otherwise
// split it into branches, which make it wait for every load in flight).
__device__ __forceinline__ const void* opaque_addr(bool use, const void* p, const void* alt) {
    uint64_t v = reinterpret_cast<uint64_t>(use ? p : alt);
    asm("" : "+v"(v));  // touches no memory (not volatile), so uniform loads around it stay scalar
    return reinterpret_cast<const void*>(v);
}

// The B operand of the down phase's matrix-core tiles.  Its 16 columns are
// (plane p, half h', activation row m) = (n >> 3, (n >> 2) & 1, n & 3): the
// hi and lo bf16 planes of the SiLU intermediate sit in columns of their own,
// so one MFMA pair per tile covers both (the dot over plane p of weight row r
// and row m, half h, is D[(r, h)][(p, h, m)]).  Four activation rows per
// pass; rows 4-7 take a second pass with the same arithmetic.  Lane l reads
// the 16 values at columns 64 h' + 16 (l >> 4) of plane p, row m.
// Adds the four parts of each (weight row, activation row) of the lanes' D
// tiles in one fixed order, ((hi, h 0) + (hi, h 1)) + ((lo, h 0) + (lo, h 1)),
// and leaves tile t's sums in LDS: red[(slot * NT + t) * 64 + r * 8 + m].
template <int NT>
__device__ __forceinline__ void planes_to_lds(const plm_f32x4 (&acc)[NT], float* red, int slot, int lane, int mbase) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = acc[t][j];
            const float hi = v + __shfl(v, (lane + 36) & 63);
            const float lo = __shfl(v, (lane + 8) & 63) + __shfl(v, (lane + 44) & 63);
            if (lane < 32 && (lane & 15) < 4)
                red[(slot * NT + t) * 64 + (4 * (lane >> 4) + j) * 8 + mbase + (lane & 3)] = hi + lo;
        }
}

template <int TT, int P, bool STAGE, bool FUSED, int MP>
__global__ __launch_bounds__(64 * kDownWaves) void fp8_down_kernel(const CombineArgs a) {
    extern __shared__ plm_u32x4 stage4[];  // STAGE: per wave, its items' activations [item][hi, lo][128] bf16
    __shared__ float red[(FUSED ? 2 : 1) * kDownWaves * TT * 64];
    __shared__ GroupInfo gi[STAGE ? 1 : kMaxGroups + 1];
    __shared__ int plan_count;
    const int nw = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int lane = threadIdx.x & 63;
    const int li = lane & 15;
    // A: the lane's weight row (li & 7) and 16 bytes at column 64 (li >> 3) + 16 (lane >> 4) of the block
    const int64_t lane_col = 64 * (li >> 3) + 16 * (lane >> 4);
    // B: column li = (plane, half, activation row); the lane's 16 values at b_col of that plane and row
    const int bplane = li >> 3, bm = li & 3;
    const int64_t b_col = 64 * ((li >> 2) & 1) + 16 * (lane >> 4);
    const unsigned char* zero = a.zero;

    int g_lo = 0, g_hi = a.ngroups, tile = blockIdx.x;
    if (a.per_group_out) {
        g_lo = tile / a.tiles_per_group;
        g_hi = g_lo + 1;
        tile -= g_lo * a.tiles_per_group;
    } else if (FUSED) {
        g_hi = a.ngroups - 1;
    }
    const int64_t row0 = static_cast<int64_t>(tile) * a.rows_per_wg;
    const int64_t rend = min(row0 + a.rows_per_wg, a.rows);
    const int64_t base = row0 & ~int64_t(7);  // tile t holds rows base + 8t .. base + 8t + 7
    int64_t roff[TT];  // rows outside [row0, rend) re-read its edge; their results are dropped
#pragma unroll
    for (int t = 0; t < TT; ++t) roff[t] = max(row0, min(base + 8 * t + (li & 7), rend - 1)) * a.K + lane_col;
    // the range spans at most two 128-row scale blocks; tile t takes the second when its rows lie there
    const int64_t srow_a = (row0 >> 7) * a.scale_cols;
    const int64_t srow_b = ((rend - 1) >> 7) * a.scale_cols;
    bool tile_b[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) tile_b[t] = ((base + 8 * t) >> 7) != (row0 >> 7);

    // The shared group's items (FUSED): blocks s_first, s_first + nw, ...
    int s_first = 0, ns = 0;
    const uint8_t* s_w = nullptr;
    const float* s_s = nullptr;
    if constexpr (FUSED) {
        const int shift = nw > a.nbe ? nw - a.nbe : 0;
        s_first = wave - shift;
        ns = s_first >= 0 ? (a.nbe - 1 - s_first) / nw + 1 : 0;
        s_w = a.w[a.ngroups - 1 - a.ndev];
        s_s = a.s[a.ngroups - 1 - a.ndev];
    }
    int nr = 0;  // routed items of this wave (blocks wave, wave + nw, ... of the summed groups), once the plan is read

    // STAGE: lane g holds group g's down matrix, scales and route weight
    // (read once by every wave at the start; items take them by readlane).
    const uint8_t* lw = nullptr;
    const float* lsc = nullptr;
    float lrw = 1.0f;
    unsigned char* region = reinterpret_cast<unsigned char*>(stage4) + static_cast<int64_t>(wave) * kDownStageItems * kDownItemBytes;

    // One pipeline slot: an item's weight tiles, its scales, its route
    // weights, whether it counts, and where its activations are.
    struct Slot {
        plm_u32x4 q[TT];
        float sv;      // lane 0: the scale of the first scale row, lane 1: of the second
        float rw[MP];  // the route weight of the lane's activation row, per pass
        bool keep[MP];
        int item;      // STAGE: the item's place in the wave's LDS region
        XPiece<true> x[MP];
    };
    auto row_live = [&](int pass) { return bm + 4 * pass < a.mc; };
    auto issue_item = [&](Slot& sl, bool exists, int g, int64_t blk, int item, const uint8_t* W, const float* S,
                          const float (&rw)[MP]) {
        bool any_keep = false;
        bool keep_l[MP];
#pragma unroll
        for (int ps = 0; ps < MP; ++ps) {
            keep_l[ps] = !(a.zero_skip && rw[ps] == 0.0f);
            any_keep = any_keep || (row_live(ps) && keep_l[ps]);
        }
        // the whole wave skips a missing item, one no live row keeps, or a group without weights
        const bool live = exists && W != nullptr && S != nullptr && __any(any_keep);
        const bool in = live && blk * 128 + lane_col < a.K;
        const int64_t col = blk * 128;
#pragma unroll
        for (int t = 0; t < TT; ++t) sl.q[t] = wload16(opaque_addr(in, W + roff[t] + col, zero + lane_col));
        // lane 0 reads the scale of the first scale row, the others that of the
        // second (a vector load, counted in order with the weights)
        sl.sv = plm_gload_f32(opaque_addr(live, S + ((lane & 1) ? srow_b : srow_a) + blk, zero));
#pragma unroll
        for (int ps = 0; ps < MP; ++ps) {
            sl.rw[ps] = rw[ps];
            // at one activation row the route weight, hence keep, is the whole wave's
            sl.keep[ps] = STAGE ? __builtin_amdgcn_readfirstlane(keep_l[ps] && live) != 0 : keep_l[ps] && live;
        }
        sl.item = item;
        if constexpr (!STAGE) {
            const bool xin = live && blk * 128 + b_col < a.K;
            const uint16_t* plane = bplane ? a.act_lo : a.act_hi;
#pragma unroll
            for (int ps = 0; ps < MP; ++ps) {
                const int m = bm + 4 * ps;
                const int64_t xo =
                    (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0 + (m < a.mc ? m : 0)) * a.K + col + b_col;
                const bool ok = xin && m < a.mc;
#pragma unroll
                for (int i = 0; i < 2; ++i) sl.x[ps].v[i] = xload16(opaque_addr(ok, plane + xo + 8 * i, zero + 16 * i));
            }
        }
    };
    auto issue_s = [&](Slot& sl, int k) {
        const bool e = k < ns;
        float rw[MP];
#pragma unroll
        for (int ps = 0; ps < MP; ++ps) rw[ps] = 1.0f;
        issue_item(sl, e, a.ngroups - 1, e ? s_first + static_cast<int64_t>(k) * nw : 0, k, e ? s_w : nullptr,
                   e ? s_s : nullptr, rw);
    };
    auto issue_r = [&](Slot& sl, int k) {
        const bool e = k < nr;
        const int c = e ? wave + k * nw : 0;
        const int gl = c / a.nbe;
        const int g = g_lo + gl;
        float rw[MP];
        if constexpr (STAGE) {
            rw[0] = e ? lane_value(lrw, g) : 1.0f;
            issue_item(sl, e, g, c - gl * a.nbe, ns + k, e ? lane_ptr(lw, g) : nullptr, e ? lane_ptr(lsc, g) : nullptr,
                       rw);
        } else {
#pragma unroll
            for (int ps = 0; ps < MP; ++ps) rw[ps] = e ? gi[g].rw[bm + 4 * ps] : 1.0f;
            issue_item(sl, e, g, c - gl * a.nbe, ns + k, e ? gi[g].w : nullptr, e ? gi[g].s : nullptr, rw);
        }
    };
    auto accumulate = [&](Slot& sl, plm_f32x4 (&acc)[MP][TT], auto san) {
        constexpr bool SAN = decltype(san)::value;
        if constexpr (STAGE) {
            if (!sl.keep[0]) return;
            // every lane reads (the item's region is written in full; lanes of
            // other activation rows feed B columns whose results are dropped)
            const unsigned char* xs = region + sl.item * kDownItemBytes + bplane * 256 + 2 * b_col;
#pragma unroll
            for (int i = 0; i < 2; ++i) sl.x[0].v[i] = *reinterpret_cast<const plm_u32x4*>(xs + 16 * i);
        }
        const float fa = lane_value(sl.sv, 0);
        const float fb = lane_value(sl.sv, 1);
        plm_bf16x8 a0[TT], a1[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) weights_to_bf16(SAN ? zero_nan_bytes(sl.q[t]) : sl.q[t], a0[t], a1[t]);
#pragma unroll
        for (int ps = 0; ps < MP; ++ps) {
            plm_bf16x8 b0, b1;
            if constexpr (SAN) {
                // infinite or NaN activations as they are (the planes carry them in hi, lo = 0)
                b0 = __builtin_bit_cast(plm_bf16x8, sl.x[ps].v[0]);
                b1 = __builtin_bit_cast(plm_bf16x8, sl.x[ps].v[1]);
            } else {
                b0 = __builtin_bit_cast(plm_bf16x8, sl.x[ps].v[0]);
                b1 = __builtin_bit_cast(plm_bf16x8, sl.x[ps].v[1]);
            }
            const float rwv = sl.rw[ps];
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                plm_f32x4 d = mfma_bf16(a0[t], b0, plm_f32x4{0.0f, 0.0f, 0.0f, 0.0f});
                d = mfma_bf16(a1[t], b1, d);
                const float f = (tile_b[t] ? fb : fa) * rwv;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if constexpr (STAGE)
                        acc[ps][t][j] = fmaf(d[j], f, acc[ps][t][j]);
                    else
                        acc[ps][t][j] = sl.keep[ps] ? fmaf(d[j], f, acc[ps][t][j]) : acc[ps][t][j];
                }
            }
        }
    };

    Slot ss, rs[P];  // the shared items' slot, the routed items' ring
    plm_f32x4 acc[MP][TT], acc_s[MP][TT];
    auto rings = [&](auto san) {
        // the shared items: the first was issued before the routed ring, so
        // waiting for it leaves the ring's loads in flight
        if (ns > 0) accumulate(ss, acc_s, san);
        for (int k = 1; k < ns; ++k) {
            issue_s(ss, k);
            accumulate(ss, acc_s, san);
        }
        for (int k0 = 0; k0 < nr; k0 += P) {
#pragma unroll
            for (int u = 0; u < P; ++u) {
                if (k0 + u < nr) accumulate(rs[u], acc, san);
                issue_r(rs[u], k0 + u + P);
            }
        }
    };
    auto zero_acc = [&]() {
#pragma unroll
        for (int ps = 0; ps < MP; ++ps)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[ps][t] = acc_s[ps][t] = plm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };
    zero_acc();

    if constexpr (STAGE) {
        // Loads in the order they are waited for: the groups' addresses and
        // route weights and the plan's count, the shared group's first item,
        // the activations of the wave's items; then the routed ring.
        int count_v = kMaxGroups + 1;
        if (lane < a.ngroups) {
            if (lane < a.ndev) {
                lw = reinterpret_cast<const uint8_t*>(a.plan->tab[4][lane]);
                lsc = reinterpret_cast<const float*>(a.plan->tab[5][lane]);
            } else {
                lw = a.w[lane - a.ndev];
                lsc = a.s[lane - a.ndev];
            }
            // one activation row, m0 (a split-off last group is unweighted and has no route entry)
            const bool routed = !(a.split_last && lane == a.ngroups - 1);
            lrw = (a.route != nullptr && routed)
                      ? a.route[static_cast<int64_t>(a.g_base + lane) * a.route_sg + static_cast<int64_t>(a.m0) * a.route_sm]
                      : 1.0f;
        }
        if (lane == 0 && a.ndev > 0) count_v = a.plan->count;
        issue_s(ss, 0);
        // the staging covers every item the groups could give this wave; the
        // plan's count is known only once the loads above are back
        const int nr_all = wave < (g_hi - g_lo) * a.nbe ? ((g_hi - g_lo) * a.nbe - 1 - wave) / nw + 1 : 0;
        const int items = ns + nr_all;  // at most kDownStageItems (the host checks)
        plm_u32x4 xv[kDownStageLoads];
        const int half = lane >> 5, plane = (lane >> 4) & 1, piece = lane & 15;
#pragma unroll
        for (int i = 0; i < kDownStageLoads; ++i) {
            const int it = 2 * i + half;
            int g, blk;
            if (it < ns) {
                g = a.ngroups - 1;
                blk = s_first + it * nw;
            } else {
                const int c = wave + (it - ns) * nw;
                g = g_lo + c / a.nbe;
                blk = c - (c / a.nbe) * a.nbe;
            }
            const bool ok = it < items && blk * 128 + piece * 8 < a.K;
            const uint16_t* src = (plane ? a.act_lo : a.act_hi) +
                                  (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0) * a.K + blk * 128 + piece * 8;
            xv[i] = xload16(opaque_addr(ok, src, zero));
        }
        const int cnt = __builtin_amdgcn_readfirstlane(count_v);
        if (a.ndev > 0) g_hi = min(g_hi, cnt);
        const int nr_items = (g_hi - g_lo) * a.nbe;
        nr = wave < nr_items ? (nr_items - 1 - wave) / nw + 1 : 0;
#pragma unroll
        for (int u = 0; u < P; ++u) issue_r(rs[u], u);
#pragma unroll
        for (int i = 0; i < kDownStageLoads; ++i)
            if (2 * i < items)
                *reinterpret_cast<plm_u32x4*>(region + (2 * i + half) * kDownItemBytes + plane * 256 + piece * 16) = xv[i];
        plm_wave_sync();
    } else {
        // The workgroup stages the groups' addresses and route weights.
        issue_s(ss, 0);
        for (int t = threadIdx.x; t < a.ngroups * kMaxM; t += blockDim.x) {
            const int g = t / kMaxM, m = t - g * kMaxM;
            if (m == 0) {
                if (g < a.ndev) {
                    gi[g].w = reinterpret_cast<const uint8_t*>(a.plan->tab[4][g]);
                    gi[g].s = reinterpret_cast<const float*>(a.plan->tab[5][g]);
                } else {
                    gi[g].w = a.w[g - a.ndev];
                    gi[g].s = a.s[g - a.ndev];
                }
            }
            const bool routed = !(a.split_last && g == a.ngroups - 1);
            gi[g].rw[m] = (a.route != nullptr && routed && m < a.mc)
                              ? a.route[static_cast<int64_t>(a.g_base + g) * a.route_sg +
                                        static_cast<int64_t>(a.m0 + m) * a.route_sm]
                              : 1.0f;
        }
        if (threadIdx.x == 0) plan_count = a.ndev > 0 ? a.plan->count : kMaxGroups + 1;
        __syncthreads();
        if (a.ndev > 0) g_hi = min(g_hi, plan_count);
        const int nr_items = (g_hi - g_lo) * a.nbe;
        nr = wave < nr_items ? (nr_items - 1 - wave) / nw + 1 : 0;
#pragma unroll
        for (int u = 0; u < P; ++u) issue_r(rs[u], u);
    }
    rings(std::false_type{});
    bool bad = false;
#pragma unroll
    for (int ps = 0; ps < MP; ++ps)
#pragma unroll
        for (int t = 0; t < TT; ++t)
#pragma unroll
            for (int j = 0; j < 4; ++j) bad = bad || acc[ps][t][j] != acc[ps][t][j] || acc_s[ps][t][j] != acc_s[ps][t][j];
    if (__any(bad)) {
        // NaN weight bytes count as 0: the wave's items again, NaN bytes zeroed
        zero_acc();
        issue_s(ss, 0);
#pragma unroll
        for (int u = 0; u < P; ++u) issue_r(rs[u], u);
        rings(std::true_type{});
    }
#pragma unroll
    for (int ps = 0; ps < MP; ++ps) {
        planes_to_lds(acc[ps], red, wave, lane, 4 * ps);
        if constexpr (FUSED) planes_to_lds(acc_s[ps], red, kDownWaves + wave, lane, 4 * ps);
    }
    __syncthreads();

    for (int t = threadIdx.x; t < TT * 64; t += blockDim.x) {
        const int tt = t >> 6, r = (t >> 3) & 7, m = t & 7;
        const int64_t row = base + 8 * tt + r;
        if (m >= a.mc || row < row0 || row >= rend) continue;
        float v = 0.0f;
        for (int w = 0; w < nw; ++w) v += red[w * TT * 64 + t];
        int64_t o = static_cast<int64_t>(a.m0 + m) * a.rows + row;
        if constexpr (FUSED) {
            float v2 = 0.0f;
            for (int w = 0; w < nw; ++w) v2 += red[(kDownWaves + w) * TT * 64 + t];
            a.out_last[o] = v2;
            a.out[o] = v;
            if (a.out_bf16 != nullptr) a.out_bf16[o] = moe_bf16_tail(v, v2, true);
        } else {
            if (a.per_group_out) o += static_cast<int64_t>(a.g_base + g_lo) * a.m_total * a.rows;
            a.out[o] = a.accumulate ? a.out[o] + v : v;
            if (a.out_bf16 != nullptr) a.out_bf16[o] = moe_bf16_tail(v, 0.0f, false);
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

// The same over the hi / lo planes of the SiLU intermediate (hi + lo is
// exact in fp32).
__device__ float scalar_plane_dot(const uint8_t* w, const float* s, const uint16_t* hi, const uint16_t* lo,
                                  int64_t K) {
    float acc = 0.0f;
    for (int64_t c0 = 0; c0 < K; c0 += 128) {
        const int64_t c1 = c0 + 128 < K ? c0 + 128 : K;
        float blk = 0.0f;
        for (int64_t c = c0; c < c1; ++c) {
            float v[4];
            plm_decode4_e4m3(static_cast<uint32_t>(w[c]), v);
            const float wv = (v[0] != v[0]) ? 0.0f : v[0];
            blk = fmaf(bf16_bits_to_f32(hi[c]) + bf16_bits_to_f32(lo[c]), wv, blk);
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
        store_hplanes(a.hhi, a.hlo, o, live ? plm_silu_mul(v[0], v[1]) : 0.0f);
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
        const int64_t xo = (static_cast<int64_t>(a.g_base + g) * a.m_total + a.m0 + m) * a.K;
        const float e = scalar_plane_dot(W + row * a.K, S + (row >> 7) * a.scale_cols, a.act_hi + xo, a.act_lo + xo,
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

// Waves per workgroup.  They split a row's K blocks (or the combine's
// items) round robin and their sums are added in wave order, so the count
// depends only on K (on the items), never on the batch: it is part of the
// per-row arithmetic.
int waves_for(int64_t items) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(items, kMaxWaves)));
}

// The rows kernel's waves for nb K blocks: preferably a count that gives
// every wave the same even number of blocks, which the pipelined loop runs
// with no unpipelined remainder (7168 columns: 56 blocks, 7 waves of 8).
int waves_for_blocks(int64_t nb) {
    if (nb <= kMaxWaves) return waves_for(nb);
    for (int w = kMaxWaves; w >= 4; --w)
        if (nb % w == 0 && (nb / w) % 2 == 0) return w;
    return kMaxWaves;
}

// Waves of a rows launch.  Each family of entry points keeps one rule for
// every batch size (it fixes the per-row arithmetic): the linear family
// (linear, dual, many) spreads K evenly for the pipelined loop, the SiLU
// gate/up phase of the MLP / MoE family takes min(4, blocks): four
// workgroups of four waves per CU instead of two of eight, so a slow wave
// holds back a smaller share of the CU (DeepSeek-V3 layer, device-routed:
// 76.9-77.8 us against 78.3-79.7 with 8 waves, same box).
constexpr int kSiluWaves = 4;
template <bool SILU>
int rows_waves(int64_t nb) {
    return SILU ? static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(nb, kSiluWaves))) : waves_for_blocks(nb);
}

// Tiles per wave (TT, 8 rows each) and blocks in flight per wave (U) only
// shape the grid and the schedule, so they are chosen per launch.  Measured
// on the DeepSeek-V3 shapes (us, one MI355X): at one activation row 1 tile
// with 2 blocks in flight (o 7168x16384 25.5, 2048x7168 6.3), and 1 tile
// in bursts for the gate/up pair (with 8 waves: bursts of 4 blocks, 9
// experts' gate/up 41.5 against 43.9 with 2 tiles and 1 block; with the 4
// waves of rows_waves, bursts of 2); with several rows, wider tiles share each
// activation load among more weight rows while the grid keeps enough
// workgroups (o at 8 rows: 4 tiles 29.5, 2 tiles 32.9, 1 tile 45.0).
constexpr int64_t kMinTiles = 192;
constexpr int64_t kCUs = 256;  // MI355X compute units

// XS: 1 when the launch has one activation row, 2 for two to four.
template <int TT, int P, bool BURST, int NWT, bool SILU, int XS = 0>
void launch_rows_cfg(const RowsArgs& a, int ngroups, hipStream_t st) {
    RowsArgs b = a;
    b.tiles_per_group = static_cast<int>(plm::ceil_div(a.rows, 8 * TT));
    const int nw = rows_waves<SILU>(a.nblocks);
    b.nw = nw;
    int64_t grid = static_cast<int64_t>(b.tiles_per_group) * ngroups + (a.inplan ? 1 : 0);
    if (a.nvar > 0) {
        b.vtile[0] = 0;
        for (int i = 0; i < a.nvar; ++i)
            b.vtile[i + 1] = b.vtile[i] + static_cast<int>(plm::ceil_div(a.vrows[i], 8 * TT));
        grid = b.vtile[a.nvar];
    }
    if constexpr (NWT == 2 && SILU) {
        if (a.inplan) {
            if (a.xb != nullptr)
                hipLaunchKernelGGL((fp8_rows_kernel<TT, P, BURST, NWT, SILU, true, true, XS>),
                                   dim3(static_cast<unsigned>(grid)), dim3(nw * plm::kWave), 0, st, b);
            else
                hipLaunchKernelGGL((fp8_rows_kernel<TT, P, BURST, NWT, SILU, false, true, XS>),
                                   dim3(static_cast<unsigned>(grid)), dim3(nw * plm::kWave), 0, st, b);
            return;
        }
    }
    if (a.xb != nullptr) {
        hipLaunchKernelGGL((fp8_rows_kernel<TT, P, BURST, NWT, SILU, true, false, XS>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    } else {
        hipLaunchKernelGGL((fp8_rows_kernel<TT, P, BURST, NWT, SILU, false, false, XS>), dim3(static_cast<unsigned>(grid)),
                           dim3(nw * plm::kWave), 0, st, b);
    }
}

// Workgroups of a rows launch at TT tiles per wave.
int64_t rows_tiles(const RowsArgs& a, int ngroups, int tt) {
    if (a.nvar == 0) return plm::ceil_div(a.rows, 8 * tt) * ngroups;
    int64_t n = 0;
    for (int i = 0; i < a.nvar; ++i) n += plm::ceil_div(a.vrows[i], 8 * tt);
    return n;
}

// Blocks per wave of a rows launch.
template <bool SILU>
int64_t rows_blocks_per_wave(const RowsArgs& a) {
    return plm::ceil_div(a.nblocks, rows_waves<SILU>(a.nblocks));
}

template <int NWT>
void launch_rows_linear(const RowsArgs& b, int mcount, int ngroups, hipStream_t st);

template <int NWT, bool SILU>
void launch_rows(const RowsArgs& a, int mcount, int ngroups, hipStream_t st) {
    RowsArgs b = a;
    b.mc = mcount;
    if constexpr (SILU) {
        // the MoE's gate/up: bursts of 2 blocks (of a wave's 14 at 7168
        // columns; bursts of 3, 4, 5 and 7 were slower)
        if (mcount == 1 || rows_tiles(b, ngroups, 2) < kMinTiles)
            launch_rows_cfg<1, 2, true, NWT, SILU>(b, ngroups, st);
        else
            launch_rows_cfg<2, 1, true, NWT, SILU>(b, ngroups, st);
    } else {
        launch_rows_linear<NWT>(b, mcount, ngroups, st);
    }
}

// The linear family's launches of several activation rows (XS 2: at most
// four; the 4-tile instance keeps its own loads: o 7168x16384 at 2 and 4
// rows was 0.4-0.6 us slower with the pair-shared halves, the 1- and 2-tile
// shapes 0.25-0.65 us faster).
template <int NWT, int XS>
void launch_rows_batch(const RowsArgs& b, int ngroups, bool few, hipStream_t st) {
    constexpr bool SILU = false;
    if constexpr (NWT == 1) {
        if (rows_tiles(b, ngroups, 4) >= kMinTiles) {
            launch_rows_cfg<4, 2, false, NWT, SILU>(b, ngroups, st);
            return;
        }
    }
    if (rows_tiles(b, ngroups, 2) >= kMinTiles) {
        launch_rows_cfg<2, 2, false, NWT, SILU, XS>(b, ngroups, st);
    } else if (few) {
        launch_rows_cfg<1, 2, false, NWT, SILU, XS>(b, ngroups, st);
    } else {
        launch_rows_cfg<1, 4, false, NWT, SILU, XS>(b, ngroups, st);
    }
}

// The linear family's launches.
template <int NWT>
void launch_rows_linear(const RowsArgs& b, int mcount, int ngroups, hipStream_t st) {
    constexpr bool SILU = false;
    // Pipeline depth at one row: every block of a wave in flight up to 8
    // (7168 columns: q_a 1536 rows 6.0 us, 576 rows 5.8, 2048 rows 6.1),
    // 4 deep beyond (16384 columns: 28.0 us against 32.2 at 8 deep).
    const int64_t per_wave = rows_blocks_per_wave<SILU>(b);
    const bool few = per_wave <= 4;  // a 4-deep pipeline would leave them unpipelined
    if (mcount == 1) {
        // short rows: wider tiles while the grid stays large (q_b 24576x1536
        // in the FP8 attention block 24.2 -> about 13 us with 4 tiles; the
        // expert down 7168x2048 6.32 -> 6.23 with 2, 6.78 with 4)
        if (few && rows_tiles(b, ngroups, 4) >= 2 * kCUs)
            launch_rows_cfg<4, 2, false, NWT, SILU, 1>(b, ngroups, st);
        else if (few && rows_tiles(b, ngroups, 2) >= kMinTiles)
            launch_rows_cfg<2, 2, false, NWT, SILU, 1>(b, ngroups, st);
        else if (few)
            launch_rows_cfg<1, 2, false, NWT, SILU, 1>(b, ngroups, st);
        else if (per_wave <= 8 && rows_tiles(b, ngroups, 1) <= plm::cu_count())
            // 8 deep holds 146 VGPRs: one workgroup per CU, so only while the grid fits the CUs
            // (q_a + kv_a, 264 tiles: 9.7 us at 8 deep)
            launch_rows_cfg<1, 8, false, NWT, SILU, 1>(b, ngroups, st);
        else
            launch_rows_cfg<1, 4, false, NWT, SILU, 1>(b, ngroups, st);
        return;
    }
    if (mcount <= 4)
        launch_rows_batch<NWT, 2>(b, ngroups, few, st);
    else
        launch_rows_batch<NWT, 0>(b, ngroups, few, st);
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

// The device address of down_zero_page on the current device (looked up the
// first time a device asks, with that device current, and kept).
int zero_page_address(const unsigned char** out) {
    static std::mutex mu;
    static std::vector<std::pair<int, const unsigned char*>> known;
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return plm::hip_fail(err, "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& k : known)
        if (k.first == dev) {
            *out = k.second;
            return 0;
        }
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(down_zero_page));
    if (err != hipSuccess) return plm::hip_fail(err, "hipGetSymbolAddress(down_zero_page)");
    known.emplace_back(dev, static_cast<const unsigned char*>(p));
    *out = static_cast<const unsigned char*>(p);
    return 0;
}

// Kernels whose LDS passes 64 KiB must say so once per device: bytes is the
// most dynamic LDS a launch of fn asks for (its static LDS comes on top).
int allow_large_lds(const void* fn, int bytes) {
    static std::mutex mu;
    static std::vector<std::pair<const void*, int>> done;
    int dev = 0;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return plm::hip_fail(err, "hipGetDevice");
    std::lock_guard<std::mutex> lock(mu);
    for (const auto& d : done)
        if (d.first == fn && d.second == dev) return 0;
    err = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess) return plm::hip_fail(err, "LDS attribute");
    done.emplace_back(fn, dev);
    return 0;
}

template <int TT, int P, bool STAGE, bool FUSED, int MP>
int launch_down_cfg(const CombineArgs& b, unsigned grid, int nw, size_t shmem, hipStream_t st) {
    const void* fn = reinterpret_cast<const void*>(&fp8_down_kernel<TT, P, STAGE, FUSED, MP>);
    if (shmem > 0) {
        const int code = allow_large_lds(fn, kDownWaves * kDownStageItems * kDownItemBytes);
        if (code != 0) return code;
    }
    hipLaunchKernelGGL((fp8_down_kernel<TT, P, STAGE, FUSED, MP>), dim3(grid), dim3(nw * plm::kWave), shmem, st, b);
    return 0;
}

template <int TT, int P, bool STAGE, int MP>
int launch_down_tt(const CombineArgs& b, unsigned grid, int nw, size_t shmem, hipStream_t st) {
    return b.fused ? launch_down_cfg<TT, P, STAGE, true, MP>(b, grid, nw, shmem, st)
                   : launch_down_cfg<TT, P, STAGE, false, MP>(b, grid, nw, shmem, st);
}

// The down phase (fp8_down_kernel): rows per workgroup so that the grid
// fills the compute units once (7168 rows: 28 each, 256 workgroups), up to
// 32; the split-off last group always in the routed workgroups (FUSED); the
// activation planes in LDS at one row when they fit.
int launch_combine(const CombineArgs& a, int mcount, hipStream_t st) {
    CombineArgs b = a;
    b.mc = mcount;
    b.fused = b.split_last ? 1 : 0;  // FUSED is the layout of a split-off last group, nothing else
    const int zc = zero_page_address(&b.zero);
    if (zc != 0) return zc;
    const int outs = b.per_group_out ? b.ngroups : 1;
    // activation rows 5-8 take a second pass of B columns (the same arithmetic
    // per row) and hold twice the accumulators: at most 16 rows per workgroup
    const int mp = mcount > 4 ? 2 : 1;
    int64_t per = plm::ceil_div(b.rows * outs, plm::cu_count());
    per = std::min<int64_t>(mp == 2 ? 16 : kDownMaxRows, std::max<int64_t>(4, plm::ceil_div(per, 4) * 4));
    b.rows_per_wg = static_cast<int>(per);
    b.tiles_per_group = static_cast<int>(plm::ceil_div(b.rows, per));
    const int nw = static_cast<int>(
        std::max<int64_t>(1, std::min<int64_t>(static_cast<int64_t>(combine_segments(b)) * b.nbe, kDownWaves)));
    const unsigned grid = static_cast<unsigned>(static_cast<int64_t>(b.tiles_per_group) * outs);
    // One activation row: each wave copies its own items' activations into
    // its LDS region (a wave's items: its shared-group blocks, then its
    // blocks of the summed groups).
    const int64_t ns_max = b.fused ? plm::ceil_div(b.nbe, nw) : 0;
    const int64_t nr_max = plm::ceil_div(static_cast<int64_t>(combine_segments(b)) * b.nbe, nw);
    const bool stage = mcount == 1 && !b.per_group_out && ns_max + nr_max <= kDownStageItems && b.K % 8 == 0 &&
                       plm::aligned16(b.act_hi) && plm::aligned16(b.act_lo);
    const size_t shmem = stage ? static_cast<size_t>(nw) * kDownStageItems * kDownItemBytes : 0;
    // Items in flight per wave within 128 VGPRs (16 waves): the activations
    // read from memory (several rows) take the registers of one slot.  At
    // 28 rows one item per wave is in flight: 16 waves of 3.5 KB items keep
    // the memory system busy, and deeper rings were slower (the 9-expert
    // DeepSeek-V3 down phase 27.0 us with 1, 33.9 with 2).
    // tiles start at multiples of 8: a range starting at 4 mod 8 takes one tile more
    const int tt = static_cast<int>(plm::ceil_div(per + (per % 8), 8));
    if (stage) {
        if (tt == 1) return launch_down_tt<1, 3, true, 1>(b, grid, nw, shmem, st);
        if (tt == 2) return launch_down_tt<2, 3, true, 1>(b, grid, nw, shmem, st);
        return launch_down_tt<4, 1, true, 1>(b, grid, nw, shmem, st);
    }
    if (mp == 2) {
        if (tt == 1) return launch_down_tt<1, 2, false, 2>(b, grid, nw, shmem, st);
        return launch_down_tt<2, 1, false, 2>(b, grid, nw, shmem, st);
    }
    if (tt == 1) return launch_down_tt<1, 3, false, 1>(b, grid, nw, shmem, st);
    if (tt == 2) return launch_down_tt<2, 2, false, 1>(b, grid, nw, shmem, st);
    return launch_down_tt<4, 1, false, 1>(b, grid, nw, shmem, st);
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
    bool tiled;           // weights in 8-row tiles (RowsArgs::tiled)
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
    if (p.tiled && (!fast || p.nvar > 0))
        return plm::fail(-2, "8-row tile weights need K %% 16 == 0 and 16-byte aligned weights and activations");
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
        const int64_t goff = static_cast<int64_t>(g0) * p.batch * p.out_ld;
        if (p.silu) {
            // the SiLU intermediate as two bf16 planes in the caller's fp32-sized buffer
            uint16_t* planes = reinterpret_cast<uint16_t*>(p.out[0]);
            a.hhi = planes + goff;
            a.hlo = planes + static_cast<int64_t>(p.ngroups) * p.batch * p.out_ld + goff;
        } else {
            for (int i = 0; i < p.nwt; ++i) a.out[i] = p.out[i] ? p.out[i] + goff : nullptr;
        }
        a.out_ld = p.out_ld;
        a.rows = p.rows;
        a.K = p.K;
        a.scale_cols = p.scale_cols;
        a.nblocks = static_cast<int>(plm::ceil_div(p.K, 128));
        a.tiled = p.tiled ? 1 : 0;
        a.m_total = static_cast<int>(p.batch);
        a.nvar = p.nvar;
        for (int i = 0; i < p.nvar; ++i) {
            a.vrows[i] = p.vrows[i];
            a.vout[i] = p.vout[i];
        }
        for (int64_t m0 = 0; m0 < p.batch; m0 += kMaxM) {
            const int mc = static_cast<int>(std::min<int64_t>(kMaxM, p.batch - m0));
            a.m0 = static_cast<int>(m0);
            a.mc = mc;
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
        a.act_hi = reinterpret_cast<const uint16_t*>(p.act);
        a.act_lo = a.act_hi + static_cast<int64_t>(p.ngroups) * p.batch * p.K;
        a.route = p.route;
        a.route_sg = p.route_sg;
        a.route_sm = p.route_sm;
        a.out = p.out;
        a.rows = p.rows;
        a.K = p.K;
        a.scale_cols = p.scale_cols;
        a.ngroups = ng;
        a.g_base = g0;
        a.nbe = static_cast<int>(plm::ceil_div(p.K, 128));
        a.per_group_out = p.per_group_out ? 1 : 0;
        a.split_last = p.out_last != nullptr ? 1 : 0;
        a.out_last = p.out_last;
        a.accumulate = (!p.per_group_out && g0 > 0) ? 1 : 0;
        a.zero_skip = p.zero_skip ? 1 : 0;
        a.m_total = static_cast<int>(p.batch);
        for (int64_t m0 = 0; m0 < p.batch; m0 += kMaxM) {
            const int mc = static_cast<int>(std::min<int64_t>(kMaxM, p.batch - m0));
            a.m0 = static_cast<int>(m0);
            a.mc = mc;
            if (fast) {
                const int lc = launch_combine(a, mc, st);
                if (lc != 0) return lc;
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
                int64_t out_rows, int64_t in_cols, int64_t scale_cols, bool tiled = false) {
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
    p.tiled = tiled;
    return run_rows(p, plm::current_stream());
}

// Bytes of a rows x cols FP8 weight in 8-row tiles: ceil(rows / 8) tile rows
// of ceil(cols / 128) tiles of 1 KB.
int64_t tiles8_bytes(int64_t rows, int64_t cols) { return plm::ceil_div(rows, 8) * plm::ceil_div(cols, 128) * 1024; }

// One thread per 16 output bytes: tile row t, block b, row r of the tile,
// piece p (16 columns), output chunk ((t * nb + b) * 8 + r) * 8 + p.  Rows
// past the matrix and columns past K are zero.
__global__ __launch_bounds__(256) void fp8_pack_tiles8_kernel(const uint8_t* __restrict__ w, uint4* __restrict__ out,
                                                              int64_t rows, int64_t cols, int64_t nb, int64_t chunks,
                                                              int vec) {
    const int64_t q = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (q >= chunks) return;
    const int64_t piece = q & 7, r = (q >> 3) & 7, tb = q >> 6;
    const int64_t b = tb % nb, t = tb / nb;
    const int64_t row = t * 8 + r, col = b * 128 + piece * 16;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < rows) {
        const uint8_t* src = w + row * cols + col;
        if (vec && col + 16 <= cols) {
            v = *reinterpret_cast<const uint4*>(src);
        } else {
            uint32_t wd[4] = {0u, 0u, 0u, 0u};
            for (int i = 0; i < 16; ++i)
                if (col + i < cols) wd[i >> 2] |= static_cast<uint32_t>(src[i]) << (8 * (i & 3));
            v = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        }
    }
    out[q] = v;
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
    uint16_t* hhi = reinterpret_cast<uint16_t*>(act);
    uint16_t* hlo = hhi + static_cast<int64_t>(groups) * batch * inter;

    RowsArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = hidden.f32;
    a.xb = hidden.bf16;
    a.x_stride = hid;
    a.hhi = hhi;
    a.hlo = hlo;
    a.out_ld = inter;
    a.rows = inter;
    a.K = hid;
    a.scale_cols = gsc;
    a.nblocks = static_cast<int>(plm::ceil_div(hid, 128));
    a.m_total = static_cast<int>(batch);
    a.mc = static_cast<int>(batch);

    int code = 0;
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
        code = plm::check_launch("moe route + plan kernel");
    } else {
        // the plan is made in the gate/up launch (its first workgroup writes
        // it; the routed workgroups find their experts from the choices)
        a.inplan = 1;
        a.pbatch = static_cast<int>(batch);
        a.ptop_k = static_cast<int>(top_k);
        a.pexperts = num_experts;
        a.ptable = table;
        a.pidx = idx;
        a.pwts = wts;
        a.pout = plan;
        a.prejected = rejected;
    }
    if (code != 0) return code;

    if (shared != nullptr) {
        a.w[0][0] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(shared[0]));
        a.s[0][0] = reinterpret_cast<const float*>(static_cast<uintptr_t>(shared[1]));
        a.w[1][0] = reinterpret_cast<const uint8_t*>(static_cast<uintptr_t>(shared[2]));
        a.s[1][0] = reinterpret_cast<const float*>(static_cast<uintptr_t>(shared[3]));
    }
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
    c.act_hi = reinterpret_cast<const uint16_t*>(act);
    c.act_lo = c.act_hi + static_cast<int64_t>(groups) * batch * inter;
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
    c.nbe = static_cast<int>(plm::ceil_div(inter, 128));
    c.m_total = static_cast<int>(batch);
    c.plan = plan;
    c.ndev = ndev;
    c.fused = 1;
    c.out_bf16 = out_bf16;
    code = launch_combine(c, static_cast<int>(batch), st);
    if (code != 0) return code;
    return plm::check_launch("fp8 down kernel");
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

PLM_EXPORT int64_t fp8_e4m3_tiles8_bytes(int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || rows > (int64_t{1} << 40) / cols) return plm::fail(-2, "bad dimensions");
    return tiles8_bytes(rows, cols);
}

PLM_EXPORT int fp8_e4m3_pack_tiles8(const uint8_t* fp8_weight, uint8_t* out_tiles, int64_t rows, int64_t cols) {
    if (!fp8_weight || !out_tiles) return plm::fail(-1, "null pointer");
    if (rows <= 0 || cols <= 0 || rows > (int64_t{1} << 40) / cols) return plm::fail(-2, "bad dimensions");
    if (!plm::aligned16(out_tiles)) return plm::fail(-2, "the tiles need a 16-byte aligned buffer");
    const int64_t nb = plm::ceil_div(cols, 128);
    const int64_t chunks = tiles8_bytes(rows, cols) / 16;
    const int vec = cols % 16 == 0 && plm::aligned16(fp8_weight);
    hipLaunchKernelGGL(fp8_pack_tiles8_kernel, dim3(static_cast<unsigned>(plm::ceil_div(chunks, 256))), dim3(256), 0,
                       plm::current_stream(), fp8_weight, reinterpret_cast<uint4*>(out_tiles), rows, cols, nb, chunks,
                       vec);
    return plm::check_launch("fp8 pack tiles8 kernel");
}

PLM_EXPORT int fp8_e4m3_block_linear_tiles8_f32(const uint8_t* fp8_tiles, const float* scale_inv, const float* hidden,
                                                float* out, int64_t batch, int64_t out_rows, int64_t in_cols,
                                                int64_t scale_cols) {
    if (!fp8_tiles || !scale_inv || !hidden || !out) return plm::fail(-1, "null pointer");
    return linear_impl(fp8_tiles, scale_inv, Act{hidden, nullptr}, out, batch, out_rows, in_cols, scale_cols, true);
}

PLM_EXPORT int fp8_e4m3_block_linear_tiles8_bf16x_f32(const uint8_t* fp8_tiles, const float* scale_inv,
                                                      const uint16_t* hidden_bf16, float* out, int64_t batch,
                                                      int64_t out_rows, int64_t in_cols, int64_t scale_cols) {
    if (!fp8_tiles || !scale_inv || !hidden_bf16 || !out) return plm::fail(-1, "null pointer");
    return linear_impl(fp8_tiles, scale_inv, Act{nullptr, hidden_bf16}, out, batch, out_rows, in_cols, scale_cols,
                       true);
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
