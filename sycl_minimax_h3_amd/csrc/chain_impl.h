// chain_impl.h - the row chain kernel behind h3s_rms_norm_mod, h3s_layer_norm (kernels/h3sycl.cpp:766-810,
// 1248-1274) and the fused h3s_norm_mod_act_gate, instantiated per input type in chain_bf16.hip, chain_f16.hip and
// chain_f32.hip.
//
// What it computes for each row (the oracle's h3o_norm_mod_act_gate; rms_norm_mod and layer_norm are the cases
// with no activation, gate or residual):
//   RMS:    n = x * inv,             inv = 1 / sqrt(sum x^2 / C + eps)
//   LAYER:  n = (x - mean) * inv,    mean = sum x / C, inv = 1 / sqrt(sum (x - mean)^2 / C + eps)
//   v = n [* w] [+ b] [* (1 + scale[t]) + shift[t]];  v = act(v) [* gate[t]];  out = [res +] v
// with t = rows[r] (table row 0 when rows is NULL), everything in float32 and one rounding to out's type. The sums
// follow the canonical order of rowcore.h. The row layout, the canonical sums and the stores are rowcore.h's; every
// load of the row (x, the residual, the weights, the table rows) is issued before the first value is used.
#pragma once

#include "rowcore.h"

namespace h3 {

struct ChainArgs {
    const void* x;
    int64_t M, C;
    int norm;                 // H3S_NORM_RMS or H3S_NORM_LAYER
    const float* w;           // NULL: no weight
    const float* b;           // NULL: no bias
    float eps;
    const int32_t* rows;      // NULL: table row 0 for every token
    const void* scale;        // scale and shift: both or neither
    const void* shift;
    const void* gate;         // NULL: 1
    int tab_dt;
    int act;
    const void* res;          // NULL: no residual
    int res_dt;
    void* out;
    int out_dt;
};

// R rows a unit: with R > 1 (rows of 256 or 512 lanes, one unit a block) the block takes rows R b .. R b + R - 1.
// It issues every row's x and residual together, loads the weights and the table rows once and uses them for all
// its rows, reloading the table rows only for a row whose table row differs. The weights and tables are read from
// L2 by every block. At 16896 x 4096 with the AdaLN's three tables, two rows a block took the chain from 74.2 to
// 70.8 us (cache-cold); three or four rows were slower (more registers, fewer wavefronts a SIMD).
// The rows of one unit: with first < 0 (R == 1) the row_pos layout (one row a block of L >= 256 lanes, or several
// rows of 64 lanes a block); else the block's rows first .. first + R - 1 (rows of 256 or 512 lanes).
template <int XDT, int CPL, int F, int R>
__device__ __forceinline__ void row_chain_rows(const ChainArgs& A, int lshift, int64_t first) {
    constexpr int V = Vec<XDT>::V;
    constexpr bool DYN = F & ROW_DYN;
    constexpr bool TW = DYN || (F & ROW_TAB32), RW = DYN || (F & ROW_RES32);   // wide storage of tables, residual
    __shared__ float red[2 * R][8];
    const bool has_w = DYN ? A.w != nullptr : (F & ROW_W) != 0;
    const bool has_b = DYN ? A.b != nullptr : (F & ROW_B) != 0;
    const bool has_tab = DYN ? A.scale != nullptr : (F & ROW_TAB) != 0;
    const bool has_gate = DYN ? A.gate != nullptr : (F & ROW_GATE) != 0;
    const bool has_res = DYN ? A.res != nullptr : (F & ROW_RES) != 0;
    // exact masks: norm and activation fixed, every 16-bit tensor bfloat16
    const int tab_dt = DYN ? A.tab_dt : (F & ROW_TAB32) ? H3S_F32 : H3S_BF16;
    const int res_dt = DYN ? A.res_dt : (F & ROW_RES32) ? H3S_F32 : H3S_BF16;
    const int out_dt = DYN ? A.out_dt : H3S_BF16;
    const int norm = DYN ? A.norm : (F & ROW_LN) ? H3S_NORM_LAYER : H3S_NORM_RMS;
    const int act_kind = DYN ? A.act : row_act(F);
    const int L = 1 << lshift;
    const int64_t C = A.C, nch = C / V;
    // this lane's place: lane t of the rows rowk[0 .. R) (clamped into [0, M); live = false past M)
    int t, W;
    int64_t rowk[R];
    bool livek[R];
    if (R == 1 && first < 0) {
        const RowPos P = row_pos(lshift, A.M);
        t = P.t;
        W = P.W;
        rowk[0] = P.row;
        livek[0] = P.live;
    } else {
        t = (int) threadIdx.x;
        W = L >> 6;
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const int64_t r = first + k;
            livek[k] = r < A.M;
            rowk[k] = livek[k] ? r : A.M - 1;
        }
    }

    // chunk j of this lane, clamped into the row (a clamped chunk is loaded and never used)
    int64_t cc[CPL];
    bool ok[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = t + (int64_t) L * j;
        ok[j] = c < nch;
        cc[j] = ok[j] ? c : nch - 1;
    }

    // ---- every load, in flight together: the rows' table row indices, then the rows and their residuals (HBM,
    // streamed once), then the weights and table rows (small, cache resident, shared by the unit's rows) ----
    const bool tabbed = (has_tab || has_gate) && A.rows;
    int64_t trk[R];
#pragma unroll
    for (int k = 0; k < R; ++k) trk[k] = tabbed ? (int64_t) A.rows[rowk[k]] * C : 0;
    int64_t tr = trk[0];
    uint4 xr[R][CPL];
    Raw<V, RW> rr[R][CPL];
#pragma unroll
    for (int k = 0; k < R; ++k) {
        const uint4* xp = reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(A.x) + rowk[k] * C * (16 / V));
#pragma unroll
        for (int j = 0; j < CPL; ++j) xr[k][j] = ld_nt(xp + cc[j]);
        if (has_res)
#pragma unroll
            for (int j = 0; j < CPL; ++j) fetch<V, RW, true>(rr[k][j], A.res, res_dt, rowk[k] * C + cc[j] * V);
    }
    Raw<V, true> wr[CPL], br[CPL];
    Raw<V, TW> sr[CPL], hr[CPL], gr[CPL];
    if (has_w)
#pragma unroll
        for (int j = 0; j < CPL; ++j) fetch(wr[j], A.w, H3S_F32, cc[j] * V);
    if (has_b)
#pragma unroll
        for (int j = 0; j < CPL; ++j) fetch(br[j], A.b, H3S_F32, cc[j] * V);
    auto load_tables = [&](int64_t at) {
        if (has_tab) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                fetch(sr[j], A.scale, tab_dt, at + cc[j] * V);
                fetch(hr[j], A.shift, tab_dt, at + cc[j] * V);
            }
        }
        if (has_gate)
#pragma unroll
            for (int j = 0; j < CPL; ++j) fetch(gr[j], A.gate, tab_dt, at + cc[j] * V);
    };
    load_tables(tr);

#pragma unroll
    for (int k = 0; k < R; ++k) {
        const int64_t row = rowk[k];
        if (k > 0 && trk[k] != tr) {
            // a row of another table row (a segment boundary between the unit's rows): its own tables
            tr = trk[k];
            load_tables(tr);
        }

        // ---- row statistics ----
        float v[CPL][V];
#pragma unroll
        for (int j = 0; j < CPL; ++j) Vec<XDT>::unpack(xr[k][j], v[j]);
        float mean = 0.0f, inv;
        if (norm == H3S_NORM_LAYER) {
            float s = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (ok[j])
#pragma unroll
                    for (int e = 0; e < V; ++e) s = s + v[j][e];
            mean = row_sum(s, red[2 * k], W) / (float) C;
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (ok[j])
#pragma unroll
                    for (int e = 0; e < V; ++e) {
                        const float d = v[j][e] - mean;
                        q = __builtin_fmaf(d, d, q);
                    }
            inv = inv_root(row_sum(q, red[2 * k + 1], W), (float) C, A.eps);
        } else {
            float q = 0.0f;
#pragma unroll
            for (int j = 0; j < CPL; ++j)
                if (ok[j])
#pragma unroll
                    for (int e = 0; e < V; ++e) q = __builtin_fmaf(v[j][e], v[j][e], q);
            inv = inv_root(row_sum(q, red[2 * k], W), (float) C, A.eps);
        }

        // ---- the chain, one chunk at a time ----
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            float o[V], f[V], g[V];
            if (norm == H3S_NORM_LAYER) {
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = (v[j][e] - mean) * inv;
            } else {
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = v[j][e] * inv;
            }
            if (has_w) {
                decode(wr[j], H3S_F32, f);
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = o[e] * f[e];
            }
            if (has_b) {
                decode(br[j], H3S_F32, f);
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = o[e] + f[e];
            }
            if (has_tab) {
                decode(sr[j], tab_dt, f);
                decode(hr[j], tab_dt, g);
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = o[e] * (1.0f + f[e]) + g[e];
            }
            if (act_kind == H3S_ACT_GELU_TANH) {
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = act_gelu_tanh(o[e]);
            } else if (act_kind == H3S_ACT_SILU) {
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = act_silu(o[e]);
            }
            if (has_gate) {
                decode(gr[j], tab_dt, f);
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = o[e] * f[e];
            }
            if (has_res) {
                decode(rr[k][j], res_dt, f);
#pragma unroll
                for (int e = 0; e < V; ++e) o[e] = f[e] + o[e];
            }
            if (livek[k] && ok[j]) store_chunk<V>(A.out, out_dt, row * C + cc[j] * V, o);
        }
    }
}

// R rows a block (R > 1: rows of 256 or 512 lanes). TAIL: the blocks from tail_blk0 on take one row each, the rows
// from tail_row0 on: a launch of two-row blocks whose last round would fill at most half the device (16896 rows of
// 4096 features: 5.5 rounds of the resident blocks) ends instead with a round of one-row blocks, twice as many and
// half as long.
template <int XDT, int CPL, int F, int R = 1, bool TAIL = false>
__global__ __launch_bounds__(512) void row_chain_kernel(ChainArgs A, int lshift, int64_t tail_blk0, int64_t tail_row0) {
    if constexpr (TAIL) {
        static_assert(R > 1, "row_chain_kernel: a tail of one-row blocks after blocks of several rows");
        if ((int64_t) blockIdx.x >= tail_blk0) {
            row_chain_rows<XDT, CPL, F, 1>(A, lshift, tail_row0 + ((int64_t) blockIdx.x - tail_blk0));
            return;
        }
    }
    row_chain_rows<XDT, CPL, F, R>(A, lshift, R == 1 ? -1 : (int64_t) blockIdx.x * R);
}

// The call shapes compiled exactly (bfloat16 rows, 16-bit tensors all bfloat16): h3s_rms_norm_mod without and with
// its float32 tables, h3s_layer_norm without and with weight and bias, and the AdaLN chain (16-bit tables, gate and
// residual) for each norm and activation. Every other call shape runs the ROW_DYN instantiation.
constexpr int kChainW = ROW_W, kChainWTab32 = ROW_W | ROW_TAB | ROW_TAB32, kChainLn = ROW_LN, kChainLnWB = ROW_LN | ROW_W | ROW_B,
              kChainAda = ROW_TAB | ROW_GATE | ROW_RES;

inline int chain_features(const ChainArgs& A, int x_dt) {
    const bool bf = x_dt == H3S_BF16 && A.out_dt == H3S_BF16 && (!(A.scale || A.gate) || A.tab_dt != H3S_F16) &&
                    (!A.res || A.res_dt == H3S_BF16);
    const int f = (A.w ? ROW_W : 0) | (A.b ? ROW_B : 0) | (A.scale ? ROW_TAB | (A.tab_dt == H3S_F32 ? ROW_TAB32 : 0) : 0) |
                  (A.gate ? ROW_GATE : 0) | (A.res ? ROW_RES : 0) | (A.norm == H3S_NORM_LAYER ? ROW_LN : 0);
    if (!bf || (A.gate && A.tab_dt == H3S_F32)) return ROW_DYN;
    if (A.act == H3S_ACT_NONE && (f == kChainW || f == kChainWTab32 || f == kChainLn || f == kChainLnWB)) return f;
    if ((f & ~ROW_LN) == kChainAda) return f | A.act * ROW_ACT1;
    return ROW_DYN;
}

// Launches the chain for one input type; the plan comes from row_plan.
template <int XDT> int chain_launch(Ctx* c, const char* fn, const ChainArgs& A, RowPlan p) {
    const RowLaunch R = row_launch(A.M, p);
    const int f = chain_features(A, XDT);
    // two rows a block: rows of 256 or 512 lanes and at most two chunks a lane (more would cost wavefronts a SIMD),
    // with side inputs the rows share, and rows enough that half as many blocks still fill the device many times
    const bool pair = XDT == H3S_BF16 && f != ROW_DYN && p.L >= 256 && p.cpl <= 2 &&
                      (f & (ROW_W | ROW_B | ROW_TAB | ROW_GATE)) && A.M >= (int64_t) c->cus * 16;
    const int64_t pairs = (A.M + 1) / 2;
    // the pairs that fill whole rounds of the device, and the rows of a last round at most half full as one-row
    // blocks
    auto tail_split = [&](const void* k, int64_t& main_blocks, int64_t& tail_blocks) {
        main_blocks = pairs;
        tail_blocks = 0;
        const int64_t round = (int64_t) c->cus * blocks_per_cu(k, (int) R.threads);
        const int64_t full = pairs / round * round;
        if (full > 0 && full < pairs && 2 * (pairs - full) <= round) {
            main_blocks = full;
            tail_blocks = A.M - 2 * full;
        }
    };
#define H3_CHAIN_F(CC, FF)                                                                                            \
    {                                                                                                                 \
        if constexpr (CC <= 2) {                                                                                      \
            if (pair) {                                                                                               \
                int64_t mb, tb;                                                                                       \
                tail_split((const void*) row_chain_kernel<XDT, CC, FF, 2, true>, mb, tb);                             \
                row_chain_kernel<XDT, CC, FF, 2, true><<<(unsigned) (mb + tb), R.threads, 0, c->stream>>>(A, R.lshift, mb, 2 * mb); \
                return launched(fn);                                                                                  \
            }                                                                                                         \
        }                                                                                                             \
        row_chain_kernel<XDT, CC, FF, 1><<<R.grid, R.threads, 0, c->stream>>>(A, R.lshift, 0, 0);                    \
    }
#define H3_CHAIN_D(CC) row_chain_kernel<XDT, CC, ROW_DYN, 1><<<R.grid, R.threads, 0, c->stream>>>(A, R.lshift, 0, 0)
#define H3_CHAIN_ADA(CC, NORM)                                                                                        \
    if (f == (kChainAda | NORM)) { H3_CHAIN_F(CC, kChainAda | NORM); return launched(fn); }                          \
    if (f == (kChainAda | NORM | H3S_ACT_GELU_TANH * ROW_ACT1)) { H3_CHAIN_F(CC, kChainAda | NORM | H3S_ACT_GELU_TANH * ROW_ACT1); return launched(fn); } \
    if (f == (kChainAda | NORM | H3S_ACT_SILU * ROW_ACT1)) { H3_CHAIN_F(CC, kChainAda | NORM | H3S_ACT_SILU * ROW_ACT1); return launched(fn); }
#define H3_CHAIN_CPL(CC)                                                                        \
    if (p.cpl == CC) {                                                                          \
        if constexpr (XDT == H3S_BF16) {                                                        \
            if (f == kChainW) { H3_CHAIN_F(CC, kChainW); return launched(fn); }                 \
            if (f == kChainWTab32) { H3_CHAIN_F(CC, kChainWTab32); return launched(fn); }       \
            if (f == kChainLn) { H3_CHAIN_F(CC, kChainLn); return launched(fn); }               \
            if (f == kChainLnWB) { H3_CHAIN_F(CC, kChainLnWB); return launched(fn); }           \
            H3_CHAIN_ADA(CC, 0)                                                                  \
            H3_CHAIN_ADA(CC, ROW_LN)                                                             \
        }                                                                                       \
        H3_CHAIN_D(CC);                                                                         \
        return launched(fn);                                                                    \
    }
    H3_CHAIN_CPL(1)
    H3_CHAIN_CPL(2)
    H3_CHAIN_CPL(3)
    H3_CHAIN_CPL(4)
#undef H3_CHAIN_CPL
#undef H3_CHAIN_ADA
#undef H3_CHAIN_D
#undef H3_CHAIN_F
    return fail(std::string(fn) + ": no kernel for this row length");
}

}  // namespace h3
