// attention.hip - h3s_attention, h3s_attention_batch (kernels/h3sycl.h:185-197, kernels/h3sycl.cpp:1433-1917) and
// h3s_attention_causal (kernels/h3sycl.h:104-108) on the kernels of attn_impl.h. The form follows the reference's
// choice: the int8 (SageAttention) form for sequences of at least H3S_SAGE_MIN_S tokens (8192) with heads of 64 or
// 128 features unless H3S_ATTN=onednn (kernels/h3sycl.cpp:1706), the 16-bit form otherwise. Any head size up to 256
// (the causal form's limit, h3sycl.cpp:877): a head runs in the kernel of 64, 128 or 256 features, zero-padded past D.
#include <cmath>
#include <cstdio>

#include "attn_impl.h"

namespace h3 {

// q of Hq heads (row stride qs) and k, v of Hkv heads (row stride kvs) prepared into aq [Hq, Sp, DK], ak [Hkv, Sp, DK]
// (int8 codes with their scales for SAGE, else half) and av [Hkv, DK, Sp] (half), DK = attn_dk(D), zero past D
// (q_in_kernel: the pipelined kernel forms q's fragments from q itself, so q is not prepared)
template <int DT>
static void prep(Ctx* c, const void* q, const void* k, const void* v, int64_t S, int64_t Sp, int64_t Hq, int64_t Hkv, int D,
                 int64_t qs_stride, int64_t kv_stride, bool sage, bool q_in_kernel, int8_t* aq, int8_t* ak, uint16_t* av,
                 float* qs, float* ks, float* km) {
    const unsigned qblocks = (unsigned) (Hq * (Sp / kAttnRows)), kvblocks = (unsigned) (Hkv * (Sp / kAttnRows));
    const int DK = attn_dk(D);
    // 16-byte rows: every tensor aligned, the strides whole numbers of 16-byte vectors, and a head of exactly 64, 128
    // or 256 features (no padding)
    const bool vec = aligned16(q) && aligned16(k) && aligned16(v) && (qs_stride * elem_size(DT)) % 16 == 0 &&
                     (kv_stride * elem_size(DT)) % 16 == 0 && D == DK;
    auto qk = [&](const void* src, int64_t stride, unsigned blocks, const float* mean, int8_t* dst, float* sc) {
#define H3_QK(SG, DD) attn_qk_prep_vec_kernel<DT, SG, DD><<<blocks, 256, 0, c->stream>>>(src, S, Sp, stride, mean, dst, sc)
        if (!vec) {
            if (sage) attn_qk_prep_kernel<DT, true><<<blocks, 256, 0, c->stream>>>(src, S, Sp, D, DK, stride, mean, dst, sc);
            else attn_qk_prep_kernel<DT, false><<<blocks, 256, 0, c->stream>>>(src, S, Sp, D, DK, stride, mean, dst, sc);
        } else if (sage) {
            if (D == 256) H3_QK(true, 256);
            else if (D == 128) H3_QK(true, 128);
            else H3_QK(true, 64);
        } else {
            if (D == 256) H3_QK(false, 256);
            else if (D == 128) H3_QK(false, 128);
            else H3_QK(false, 64);
        }
#undef H3_QK
    };
    if (sage) {
        // k's mean per (head, feature) of the D features; the 16-byte form takes 16 features a block, or 32 where 16
        // would make more blocks than the device runs at once
        const int64_t hd = Hkv * D;
        const bool wide = hd % kKmeanFeatWide == 0 && hd / kKmeanFeat > c->cus;
        if (vec && wide) attn_kmean_kernel<DT, kKmeanFeatWide><<<(unsigned) (hd / kKmeanFeatWide), 256, 0, c->stream>>>(k, S, kv_stride, km);
        else if (vec && hd % kKmeanFeat == 0) attn_kmean_kernel<DT, kKmeanFeat><<<(unsigned) (hd / kKmeanFeat), 256, 0, c->stream>>>(k, S, kv_stride, km);
        else attn_kmean_rows_kernel<DT><<<(unsigned) ((hd + 255) / 256), 256, 0, c->stream>>>(k, S, hd, kv_stride, km);
        if (!q_in_kernel) qk(q, qs_stride, qblocks, nullptr, aq, qs);
        qk(k, kv_stride, kvblocks, km, ak, ks);
    } else {
        if (!q_in_kernel) qk(q, qs_stride, qblocks, nullptr, aq, nullptr);
        qk(k, kv_stride, kvblocks, nullptr, ak, nullptr);
    }
    if (!vec) attn_v_prep_kernel<DT><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, D, DK, kv_stride, av);
    else if (D == 256) attn_v_prep_vec_kernel<DT, 256><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, kv_stride, av);
    else if (D == 128) attn_v_prep_vec_kernel<DT, 128><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, kv_stride, av);
    else attn_v_prep_vec_kernel<DT, 64><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, kv_stride, av);
}

// one sequence: S query rows of Hq heads (row stride qs_stride) over S key/value rows of Hkv heads (kv_stride);
// causal: query i sees keys 0 .. i (the 16-bit form, as the reference's causal kernel computes in float)
static int attention_one(Ctx* c, const char* fn, const void* q, const void* k, const void* v, int dt, int64_t S, int64_t Hq,
                         int64_t Hkv, int64_t D, int64_t qs_stride, int64_t kv_stride, void* out, int out_dt, bool causal) {
    // the int8 form as the reference takes it (kernels/h3sycl.cpp:1706): heads of 64 or 128 features, and S * D * H
    // within int32; every other call runs the 16-bit form
    const bool sage = !causal && c->sage_want && S >= c->sage_min_s && (D == 64 || D == 128) && S <= INT32_MAX / D / Hq;
    // heads of 128 features into an aligned out, no causal mask: the pipelined kernel (256 queries a block)
    const bool pp = !causal && D == 128 && aligned16(out) && S <= (int64_t) kAttnPPTiles * kAttnRows;
    const int64_t qblock = pp ? kAttnPPQ : kAttnQBlock;
    const int64_t Sp = (S + qblock - 1) / qblock * qblock, nbp = Sp / kAttnRows;
    const int64_t esz = sage ? 1 : 2, DK = attn_dk(D);
    if (Hq * (Sp / qblock) > 0x7fffffff) return fail(std::string(fn) + ": too many query blocks");
    // the pipelined kernel reads q's rows itself where they are whole 16-byte vectors (no prepared q then)
    const bool q_in_kernel = pp && aligned16(q) && (qs_stride * elem_size(dt)) % 16 == 0;
    int8_t* aq = q_in_kernel ? nullptr : c->scratch<int8_t>(Ctx::ATT_Q, (size_t) (Sp * Hq * DK * esz));
    int8_t* ak = c->scratch<int8_t>(Ctx::ATT_K, (size_t) (Sp * Hkv * DK * esz));
    uint16_t* av = c->scratch<uint16_t>(Ctx::ATT_V, (size_t) (Sp * Hkv * DK));
    float* af = c->scratch<float>(Ctx::ATT_AUX, (size_t) ((Hq + Hkv) * nbp + Hkv * D));
    if ((!aq && !q_in_kernel) || !ak || !av || !af) return -1;
    float *qs = af, *ks = af + Hq * nbp, *km = af + (Hq + Hkv) * nbp;
    PhaseTimer timer(c);
    timer.mark();
    switch (dt) {
        case H3S_BF16: prep<H3S_BF16>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, q_in_kernel, aq, ak, av, qs, ks, km); break;
        case H3S_F16: prep<H3S_F16>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, q_in_kernel, aq, ak, av, qs, ks, km); break;
        default: prep<H3S_F32>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, q_in_kernel, aq, ak, av, qs, ks, km); break;
    }
    if (launched(fn)) return -1;
    AttnArgs P;
    P.q = aq; P.k = ak; P.vt = av; P.qs = qs; P.ks = ks;
    P.S = S; P.Sp = Sp; P.H = Hq;
    P.c = (float) (1.4426950408889634 * (double) (1.0f / std::sqrt((float) D)));
    P.out = out; P.out_dt = out_dt; P.D = (int) D;
    P.nqb = (int) (Sp / qblock);
    P.kvdiv = (int) (Hq / Hkv);
    P.Spk = Sp;
    P.qraw = q_in_kernel ? q : nullptr;
    P.qstride = qs_stride;
    P.q_dt = dt;
    const int64_t nblocks = Hq * P.nqb;
    P.nfull = nblocks; P.nsplit = 1; P.ts = 0; P.po = nullptr; P.pml = nullptr;
    // the pipelined kernel's last round: when it would fill at most half the CUs, its blocks each become up to
    // c->attn_split blocks of consecutive key tiles, whose results attn_merge_kernel combines
    int64_t tail = 0;
    if (pp) {
        const int64_t cus = c->cus, T = (S + kAttnRows - 1) / kAttnRows, last = nblocks % cus;
        const int64_t want = std::min<int64_t>({(int64_t) c->attn_split, last ? cus / last : 1, T});
        if (last > 0 && 2 * last <= cus && want > 1) {
            const int64_t ts = (T + want - 1) / want, ns = (T + ts - 1) / ts;
            // (no room for the partial sums under the memory cap: the last round runs unsplit)
            if (ns > 1 && (P.po = c->scratch<float>(Ctx::ATT_PART, (size_t) (last * ns * kAttnPPQ * (128 + 2))))) {
                P.pml = P.po + last * ns * kAttnPPQ * 128;
                tail = last;
                P.nfull = nblocks - last; P.nsplit = (int) ns; P.ts = (int) ts;
            }
        }
    }
    const unsigned grid = (unsigned) (P.nfull + tail * P.nsplit);
    timer.mark();
    // heads of 64, 128 or 256 features into an aligned out take the plain stores; others the masked ones
    const bool pad = D != DK || !aligned16(out);
#define H3_ATTN_D(SG, DD, CA)                                                                  \
    {                                                                                          \
        if (pad) attn_kernel<SG, DD, CA, true><<<grid, 256, 0, c->stream>>>(P);               \
        else attn_kernel<SG, DD, CA, false><<<grid, 256, 0, c->stream>>>(P);                  \
    }
#define H3_ATTN(SG, CA)                                                                        \
    {                                                                                          \
        if (DK == 256) H3_ATTN_D(SG, 256, CA)                                                  \
        else if (DK == 128) H3_ATTN_D(SG, 128, CA)                                             \
        else H3_ATTN_D(SG, 64, CA)                                                             \
    }
    if (pp) {
        if (sage) attn_pl_kernel<true, 4><<<grid, 512, 0, c->stream>>>(P);
        else attn_pl_kernel<false, 4><<<grid, 512, 0, c->stream>>>(P);
        if (tail) attn_merge_kernel<<<(unsigned) ((tail * kAttnPPQ * 32 + 255) / 256), 256, 0, c->stream>>>(P, tail);
    } else if (causal) H3_ATTN(false, true)
    else if (sage) {
        // (the int8 form only at 64 or 128 features, above)
        if (DK == 128) H3_ATTN_D(true, 128, false)
        else H3_ATTN_D(true, 64, false)
    } else H3_ATTN(false, false)
#undef H3_ATTN
#undef H3_ATTN_D
    if (launched(fn)) return -1;
    timer.mark();
    const std::vector<float> ms = timer.elapsed();
    if (ms.size() == 2)   // H3S_PROFILE (kernels/h3sycl.cpp:1753-1760)
        std::fprintf(stderr, "h3hip: attention (%s) S=%lld H=%lld D=%lld: preparation %.2f ms, attention %.2f ms\n",
                     sage ? "int8" : causal ? "16-bit, causal" : "16-bit", (long long) S, (long long) Hq, (long long) D, ms[0],
                     ms[1]);
    return 0;
}

static int attention_checks(const char* fn, int dt, int64_t H, int64_t D, int64_t stride, int out_dt, const void* q,
                            const void* k, const void* v, const void* out) {
    if (stride < H * D) return fail(std::string(fn) + ": the row stride is shorter than a row");
    if (!dt_ok(dt) || !dt_ok(out_dt)) return fail(std::string(fn) + ": unknown element type");
    if (D > kAttnMaxD) return fail(std::string(fn) + ": head size " + std::to_string(D) + " (at most 256)");
    if (!q || !k || !v || !out) return fail(std::string(fn) + ": q, k, v and out are required");
    return 0;
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_attention(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t S, int64_t H, int64_t D,
                             int64_t stride, void* out, int out_dt) try {
    const char* fn = "h3s_attention";
    if (S <= 0 || H <= 0 || D <= 0) return 0;
    if (attention_checks(fn, dt, H, D, stride, out_dt, q, k, v, out)) return -1;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return attention_one(c, fn, q, k, v, dt, S, H, H, D, stride, stride, out, out_dt, false);
} catch (const std::exception& e) { return fail(e.what()); }

// B sequences of S tokens: sequence b's rows start at row b S of q, k, v and out (kernels/h3sycl.cpp:1800-1815)
H3S_EXPORT int h3s_attention_batch(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t B, int64_t S,
                                   int64_t H, int64_t D, int64_t stride, void* out, int out_dt) try {
    const char* fn = "h3s_attention_batch";
    if (B <= 0 || S <= 0 || H <= 0 || D <= 0) return 0;
    if (attention_checks(fn, dt, H, D, stride, out_dt, q, k, v, out)) return -1;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const size_t ei = (size_t) elem_size(dt), eo = (size_t) elem_size(out_dt);
    for (int64_t b = 0; b < B; ++b) {
        const size_t io = (size_t) (b * S * stride) * ei, oo = (size_t) (b * S * H * D) * eo;
        if (attention_one(c, fn, (const char*) q + io, (const char*) k + io, (const char*) v + io, dt, S, H, H, D, stride,
                          stride, (char*) out + oo, out_dt, false))
            return -1;
    }
    return 0;
} catch (const std::exception& e) { return fail(e.what()); }

// The text encoder's causal attention with grouped key/value heads (kernels/h3sycl.h:104-108, kernels/h3sycl.cpp:873-898):
// q rows of stride qs (Hq heads), k and v rows of stride kvs (Hkv heads), head h reads kv head h / (Hq / Hkv); out
// [L, Hq * D] in dt. The 16-bit form with a causal mask; any head size up to 256, as the reference.
H3S_EXPORT int h3s_attention_causal(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t L, int64_t Hq,
                                    int64_t Hkv, int64_t D, int64_t qs, int64_t kvs, void* out) try {
    const char* fn = "h3s_attention_causal";
    if (L <= 0 || D <= 0) return 0;
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0) return fail(std::string(fn) + ": Hq must be a multiple of Hkv");
    if (D > kAttnMaxD) return fail(std::string(fn) + ": D <= 256, Hq a multiple of Hkv (head size " + std::to_string(D) + ")");
    if (qs < Hq * D || kvs < Hkv * D) return fail(std::string(fn) + ": a row stride is shorter than a row");
    if (!dt_ok(dt)) return fail(std::string(fn) + ": unknown element type");
    if (!q || !k || !v || !out) return fail(std::string(fn) + ": q, k, v and out are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return attention_one(c, fn, q, k, v, dt, L, Hq, Hkv, D, qs, kvs, out, dt, true);
} catch (const std::exception& e) { return fail(e.what()); }
