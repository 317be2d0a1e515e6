// attention.hip - h3s_attention, h3s_attention_batch (kernels/h3sycl.h:185-197, kernels/h3sycl.cpp:1433-1917) and
// h3s_attention_causal (kernels/h3sycl.h:104-108) on the kernels of attn_impl.h. The form follows the reference's choice: the int8 (SageAttention) form for sequences of
// at least H3S_SAGE_MIN_S tokens (8192) unless H3S_ATTN=onednn, the 16-bit form otherwise. Head sizes 64 and 128.
#include <cmath>
#include <cstdio>

#include "attn_impl.h"

namespace h3 {

// q of Hq heads (row stride qs) and k, v of Hkv heads (row stride kvs) prepared into aq [Hq, Sp, D], ak [Hkv, Sp, D]
// (int8 codes with their scales for SAGE, else half) and av [Hkv, D, Sp] (half)
template <int DT>
static void prep(Ctx* c, const void* q, const void* k, const void* v, int64_t S, int64_t Sp, int64_t Hq, int64_t Hkv, int D,
                 int64_t qs_stride, int64_t kv_stride, bool sage, int8_t* aq, int8_t* ak, uint16_t* av, float* qs, float* ks,
                 float* km) {
    const unsigned qblocks = (unsigned) (Hq * (Sp / kAttnRows)), kvblocks = (unsigned) (Hkv * (Sp / kAttnRows));
    // 16-byte rows: every tensor aligned and the strides whole numbers of 16-byte vectors
    const bool vec = aligned16(q) && aligned16(k) && aligned16(v) && (qs_stride * elem_size(DT)) % 16 == 0 &&
                     (kv_stride * elem_size(DT)) % 16 == 0;
    auto qk = [&](const void* src, int64_t stride, unsigned blocks, const float* mean, int8_t* dst, float* sc) {
#define H3_QK(SG, DD) attn_qk_prep_vec_kernel<DT, SG, DD><<<blocks, 256, 0, c->stream>>>(src, S, Sp, stride, mean, dst, sc)
        if (!vec) {
            if (sage) attn_qk_prep_kernel<DT, true><<<blocks, 256, 0, c->stream>>>(src, S, Sp, D, stride, mean, dst, sc);
            else attn_qk_prep_kernel<DT, false><<<blocks, 256, 0, c->stream>>>(src, S, Sp, D, stride, mean, dst, sc);
        } else if (sage) {
            if (D == 128) H3_QK(true, 128);
            else H3_QK(true, 64);
        } else {
            if (D == 128) H3_QK(false, 128);
            else H3_QK(false, 64);
        }
#undef H3_QK
    };
    if (sage) {
        const int64_t hd = Hkv * D;
        if (vec) attn_kmean_kernel<DT><<<(unsigned) (hd / kKmeanFeat), 256, 0, c->stream>>>(k, S, kv_stride, km);
        else attn_kmean_rows_kernel<DT><<<(unsigned) ((hd + 255) / 256), 256, 0, c->stream>>>(k, S, hd, kv_stride, km);
        qk(q, qs_stride, qblocks, nullptr, aq, qs);
        qk(k, kv_stride, kvblocks, km, ak, ks);
    } else {
        qk(q, qs_stride, qblocks, nullptr, aq, nullptr);
        qk(k, kv_stride, kvblocks, nullptr, ak, nullptr);
    }
    if (!vec) attn_v_prep_kernel<DT><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, D, kv_stride, av);
    else if (D == 128) attn_v_prep_vec_kernel<DT, 128><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, kv_stride, av);
    else attn_v_prep_vec_kernel<DT, 64><<<kvblocks, 256, 0, c->stream>>>(v, S, Sp, kv_stride, av);
}

// one sequence: S query rows of Hq heads (row stride qs_stride) over S key/value rows of Hkv heads (kv_stride);
// causal: query i sees keys 0 .. i (the 16-bit form, as the reference's causal kernel computes in float)
static int attention_one(Ctx* c, const char* fn, const void* q, const void* k, const void* v, int dt, int64_t S, int64_t Hq,
                         int64_t Hkv, int64_t D, int64_t qs_stride, int64_t kv_stride, void* out, int out_dt, bool causal) {
    const bool sage = !causal && c->sage_want && S >= c->sage_min_s;
    const int64_t Sp = (S + kAttnQBlock - 1) / kAttnQBlock * kAttnQBlock, nbp = Sp / kAttnRows;
    const int64_t esz = sage ? 1 : 2;
    if (Hq * (Sp / kAttnQBlock) > 0x7fffffff) return fail(std::string(fn) + ": too many query blocks");
    int8_t* aq = c->scratch<int8_t>(Ctx::ATT_Q, (size_t) (Sp * Hq * D * esz));
    int8_t* ak = c->scratch<int8_t>(Ctx::ATT_K, (size_t) (Sp * Hkv * D * esz));
    uint16_t* av = c->scratch<uint16_t>(Ctx::ATT_V, (size_t) (Sp * Hkv * D));
    float* af = c->scratch<float>(Ctx::ATT_AUX, (size_t) ((Hq + Hkv) * nbp + Hkv * D));
    if (!aq || !ak || !av || !af) return -1;
    float *qs = af, *ks = af + Hq * nbp, *km = af + (Hq + Hkv) * nbp;
    PhaseTimer timer(c);
    timer.mark();
    switch (dt) {
        case H3S_BF16: prep<H3S_BF16>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, aq, ak, av, qs, ks, km); break;
        case H3S_F16: prep<H3S_F16>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, aq, ak, av, qs, ks, km); break;
        default: prep<H3S_F32>(c, q, k, v, S, Sp, Hq, Hkv, (int) D, qs_stride, kv_stride, sage, aq, ak, av, qs, ks, km); break;
    }
    if (launched(fn)) return -1;
    AttnArgs P;
    P.q = aq; P.k = ak; P.vt = av; P.qs = qs; P.ks = ks;
    P.S = S; P.Sp = Sp; P.H = Hq;
    P.c = (float) (1.4426950408889634 * (double) (1.0f / std::sqrt((float) D)));
    P.out = out; P.out_dt = out_dt;
    P.nqb = (int) (Sp / kAttnQBlock);
    P.kvdiv = (int) (Hq / Hkv);
    P.Spk = Sp;
    const unsigned grid = (unsigned) (Hq * P.nqb);
    timer.mark();
    if (causal) {
        if (D == 128) attn_kernel<false, 128, true><<<grid, 256, 0, c->stream>>>(P);
        else attn_kernel<false, 64, true><<<grid, 256, 0, c->stream>>>(P);
    } else if (sage) {
        if (D == 128) attn_kernel<true, 128><<<grid, 256, 0, c->stream>>>(P);
        else attn_kernel<true, 64><<<grid, 256, 0, c->stream>>>(P);
    } else {
        if (D == 128) attn_kernel<false, 128><<<grid, 256, 0, c->stream>>>(P);
        else attn_kernel<false, 64><<<grid, 256, 0, c->stream>>>(P);
    }
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
    if (D != 64 && D != 128) return fail(std::string(fn) + ": head size " + std::to_string(D) + " (64 or 128 only)");
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
// [L, Hq * D] in dt. The 16-bit form with a causal mask; head sizes 64 and 128 (the reference takes D <= 256).
H3S_EXPORT int h3s_attention_causal(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t L, int64_t Hq,
                                    int64_t Hkv, int64_t D, int64_t qs, int64_t kvs, void* out) try {
    const char* fn = "h3s_attention_causal";
    if (L <= 0) return 0;
    if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0) return fail(std::string(fn) + ": Hq must be a multiple of Hkv");
    if (D != 64 && D != 128) return fail(std::string(fn) + ": head size " + std::to_string(D) + " (64 or 128 only)");
    if (qs < Hq * D || kvs < Hkv * D) return fail(std::string(fn) + ": a row stride is shorter than a row");
    if (!dt_ok(dt)) return fail(std::string(fn) + ": unknown element type");
    if (!q || !k || !v || !out) return fail(std::string(fn) + ": q, k, v and out are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    return attention_one(c, fn, q, k, v, dt, L, Hq, Hkv, D, qs, kvs, out, dt, true);
} catch (const std::exception& e) { return fail(e.what()); }
