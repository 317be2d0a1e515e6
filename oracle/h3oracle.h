/* h3oracle.h - CPU restatement of the reference's per-token layer arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: the tests, the smoke check and the CPU-baseline leg of the
 * benchmark load it to compute what the GPU library must produce. Nothing in the product path (libh3hip.so and the
 * sycl_minimax_h3_amd package) links, loads or calls it.
 *
 * Every function names the reference file:line it restates. Floating-point order is canonical: where the reference
 * leaves the order of a reduction to the device (sycl::reduce_over_group), this file fixes it, and the HIP kernels
 * follow the same order, so that results can be compared bit for bit. The canonical row reduction:
 *
 *   the row's n values are cut into chunks of V consecutive values; chunk c belongs to lane c % L;
 *   each lane accumulates its values in increasing index order, starting from +0.0f;
 *   up to L = 64 (one wavefront), the L lane partials are then combined by an xor butterfly with offsets
 *   L/2, L/4, ..., 1 (partial[l] = partial[l] + partial[l ^ off]), which leaves the same value in every lane;
 *   lane 0's is the sum. For L = 128 .. 512 (several wavefronts on one row) that butterfly runs inside each group
 *   of 64 lanes, and the L/64 group sums are then combined by the same butterfly.
 *
 * Rows of the row-wise operations (norms, fused chains) use L = h3o_row_lanes(n, V): 64 lanes below 256 chunks,
 * 256 up to 1024 chunks, 512 up to 2048.
 *
 * Squares are accumulated with a fused multiply-add (acc = fma(x, x, acc)). Everything else is written out
 * operation by operation and must be compiled with -ffp-contract=off.
 *
 * Element types follow kernels/h3sycl.h:20 (H3S_F32 = 0, H3S_F16 = 1, H3S_BF16 = 2).
 */
#ifndef H3ORACLE_H
#define H3ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { H3O_F32 = 0, H3O_F16 = 1, H3O_BF16 = 2 };
/* rotations of a group of g features (kernels/h3sycl.h:74-83 defines only the regular one) */
enum { H3O_ROT_NONE = 0, H3O_ROT_REGULAR = 1, H3O_ROT_SYLVESTER = 2 };
/* pointwise activations */
enum { H3O_ACT_NONE = 0, H3O_ACT_GELU_TANH = 1, H3O_ACT_SILU = 2 };
/* row norms of the fused modulate chain */
enum { H3O_NORM_RMS = 0, H3O_NORM_LAYER = 1 };
/* reduction kinds of h3o_canon_sum */
enum { H3O_SUM = 0, H3O_SUMSQ = 1, H3O_SUMSQ_DIFF = 2 };

/* threads for the row-parallel functions (contiguous row chunks, as engine/h3-core/src/reference.rs:43-80) */
void h3o_set_threads(int n);
int h3o_get_threads(void);

/* ---- element types: engine/h3-core/src/dtype.rs:53-121, kernels/h3sycl.cpp:42-49 ---- */
float h3o_bf16_to_f32(uint16_t b);
uint16_t h3o_f32_to_bf16(float f);
float h3o_f16_to_f32(uint16_t h);
uint16_t h3o_f32_to_f16(float f);
float h3o_load(const void* p, int dt, int64_t i);
void h3o_store(void* p, int dt, int64_t i, float v);
/* round a float32 to type dt and back (dt = F32: unchanged) */
float h3o_round_to(float v, int dt);

/* ---- seeded inputs: engine/h3-core/src/rng.rs:9-43 ---- */
typedef struct { uint64_t s[4]; } h3o_rng;
void h3o_rng_new(h3o_rng* r, uint64_t seed);
void h3o_rng_from_state(h3o_rng* r, const uint64_t s[4]);
uint64_t h3o_rng_next_u64(h3o_rng* r);
float h3o_rng_uniform(h3o_rng* r);
float h3o_rng_normal(h3o_rng* r);
/* n draws of scale * normal(), stored in type dt (engine/h3d/src/jobs.rs:92-101 does this with scale 0.7, bf16) */
void h3o_fill_normal(uint64_t seed, float scale, int64_t n, void* out, int dt);
/* n draws of lo + (hi - lo) * uniform() as float32 */
void h3o_fill_uniform(uint64_t seed, float lo, float hi, int64_t n, float* out);
/* k distinct indices of [0, n), in draw order (a partial Fisher-Yates shuffle driven by next_u64) */
void h3o_choose(uint64_t seed, int64_t n, int64_t k, int64_t* out);

/* ---- canonical reduction (see the header comment) ---- */
float h3o_canon_sum(const float* x, int64_t n, int V, int L, int kind, float mean);
/* lanes per row of n values in chunks of V (see the header comment) */
int h3o_row_lanes(int64_t n, int V);

/* ---- the reference's operations (kernels/h3sycl.h) ---- */
/* kernels/h3sycl.h:96-101, 162-163; kernels/h3sycl.cpp:766-810 */
int h3o_rms_norm_mod(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps, const int32_t* rows,
                     const float* scale, const float* shift, void* out, int out_dt);
/* kernels/h3sycl.h:159-161; kernels/h3sycl.cpp:1248-1274 */
int h3o_layer_norm(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, const float* bias, float eps,
                   void* out, int out_dt);
/* kernels/h3sycl.h:165-174; kernels/h3sycl.cpp:1276-1376 */
int h3o_rms_rope(void* x, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride, const float* weight, float eps,
                 const float* cs, int rot_dim);
/* kernels/h3sycl.h:176-178; kernels/h3sycl.cpp:1378-1419 */
int h3o_swiglu(const void* x, int x_dt, int64_t M, int64_t C, void* out, int out_dt);
/* kernels/h3sycl.h:180-183; kernels/h3sycl.cpp:1421-1431 */
int h3o_gate_add(void* x, int x_dt, int64_t M, int64_t C, const void* other, int other_dt, const int32_t* rows,
                 const float* gate);
/* kernels/h3sycl.h:74-85; kernels/h3sycl.cpp:404-652; engine/h3-core/src/reference.rs:37-82 */
int h3o_int8_linear(const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N, const float* wscale,
                    int64_t n_wscale, const float* bias, void* out, int out_dt, int group);

/* ---- the pieces of the int8 linear ---- */
/* y[g] rotated in place: regular (g = 4^k, kernels/h3sycl.cpp:433-459) or Sylvester (g = 2^k) */
void h3o_rotate_group(float* y, int g, int kind);
/* dense normalized matrices for checks: regular (engine/h3-core/src/reference.rs:4-23), Sylvester H2^(x)k / sqrt(g) */
void h3o_hadamard_regular(int g, float* h);
void h3o_hadamard_sylvester(int g, float* h);
/* per-row quantization of float32 rows (kernels/h3sycl.h:74-83, engine/h3-core/src/reference.rs:68-70) */
void h3o_quantize_rows(const float* y, int64_t M, int64_t K, int8_t* q, float* s);
/* out = act(acc * s_r * wscale + bias) from int8 codes (kernels/h3sycl.cpp:576-629, reference.rs:72-76) */
int h3o_gemm_dequant(const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N, const float* wscale,
                     int64_t n_wscale, const float* bias, int act, void* out, int out_dt);

/* ---- fused chains: compositions of the operations above ---- */
/* rms_norm_mod into a virtual h in h_dt, then the int8 linear's quantizer with an optional rotation.
 * scale/shift tables [R, C] in tab_dt (F32 or BF16); rows NULL: every token uses table row 0; scale or shift NULL:
 * no modulation. */
int h3o_norm_quant(const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps, const int32_t* rows,
                   const void* scale, const void* shift, int tab_dt, int h_dt, int rot, int group, int8_t* q, float* s);
/* h3o_swiglu into a scratch of h_dt, then the quantizer of h3o_norm_quant (rotation rot/group) on it */
int h3o_swiglu_quant(const void* x, int x_dt, int64_t M, int64_t C, int h_dt, int rot, int group, int8_t* q, float* s);
/* the quantizer alone on x [M, C]: rotation rot/group, then s = max(max|y| / 127, 1e-30), q = rint(y / s) */
int h3o_quantize_act(const void* x, int x_dt, int64_t M, int64_t C, int rot, int group, int8_t* q, float* s);
/* out = res + gate * act(norm(x) * (1 + scale) + shift): norm RMS (weight) or layer norm (weight, bias optional);
 * tables as above, gate NULL: 1; res NULL: 0. */
int h3o_norm_mod_act_gate(const void* x, int x_dt, int64_t M, int64_t C, int norm, const float* weight,
                          const float* bias, float eps, const int32_t* rows, const void* scale, const void* shift,
                          const void* gate, int tab_dt, int act, const void* res, int res_dt, void* out, int out_dt);
/* the pointwise activations, float32 */
float h3o_act(float v, int act);
void h3o_act_n(const float* v, int64_t n, int act, float* out);   /* h3o_act on each of n values */

/* ---- attention (kernels/h3sycl.h:185-192; kernels/h3sycl.cpp:1433-1917) ----
 * out = softmax(q . k^T / sqrt(D)) . v per head; q, k, v: S rows of H heads x D features at row stride `stride`
 * (elements) in dt; out [S, H * D] in out_dt.
 * sage != 0: the reference's default for S >= 8192 (h3sycl.cpp:1676-1767): k's mean over the sequence per (head,
 *   feature) taken out (a float32 sum in token order / S), q and k - mean to int8 with one scale per head per 64
 *   rows (m = the block's max |x|, code = clamp(round_half_away(x * fl(127 / m)), -127, 127), scale = m / 127), v in
 *   IEEE half; scores from the exact integer products times qscale, kscale and fl(1 / sqrt(D)).
 * sage == 0: the 16-bit form (h3sycl.cpp:1496-1550): q, k and v in IEEE half, scores times fl(1 / sqrt(D)).
 * Both: the softmax and the weighted sum in float64 (the reference's kernels are third-party: oneDNN and Intel's
 * ARK, whose internal rounding is not restated), the result rounded to half (the reference's ao buffer), then
 * stored in out_dt. The int8 codes and scales of the sage form are written to iq, ik [H, S, D], qs, ks [H, nb]
 * and kmean [H, D] when those are not NULL. */
int h3o_attention(const void* q, const void* k, const void* v, int dt, int64_t S, int64_t H, int64_t D, int64_t stride,
                  void* out, int out_dt, int sage, int8_t* iq, int8_t* ik, float* qs, float* ks, float* kmean);
/* causal attention with grouped key/value heads (kernels/h3sycl.cpp:873-898): query i of head h sees keys 0 .. i of
 * kv head h / (Hq / Hkv); q rows of stride qs, k and v rows of stride kvs, all in dt; out [L, Hq * D] in dt; the
 * softmax in float64 on the dt values, one rounding to dt. */
int h3o_attention_causal(const void* q, const void* k, const void* v, int dt, int64_t L, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t qs, int64_t kvs, void* out);
/* the sage form's quantization of one tensor: mean NULL for q; codes [H, S, D], scales [H, ceil(S / 64)] */
void h3o_sage_quantize(const void* src, int dt, int64_t S, int64_t H, int64_t D, int64_t stride, const float* mean,
                       int8_t* codes, float* scales);

/* ---- plain linear layers (kernels/h3sycl.h:87-93; kernels/h3sycl.cpp:656-739) ----
 * out [M, N] = x [M, K] . w^T (w [N, K]) + bias, x and w in dt, the products summed in float64 and rounded once to
 * out_dt; acc != 0: out = round(product + bias + out) in dt (h3s_linear_acc). The reference's matmul is oneDNN's,
 * whose accumulation order is not restated. scale_rows: x[r, i] = round(x[r, i] * s[r]). */
void h3o_linear(const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N, const float* bias, void* out,
                int out_dt, int acc);
void h3o_scale_rows(void* x, int dt, int64_t M, int64_t C, const float* s);

/* ---- a step's tables (engine/h3-core/src/dit.rs:155-203) ----
 * adaln_tables: the six AdaLN tables of one block for R timestep embeddings t_emb [R, t_dim]:
 *   out[ci][(r * m + mi) * C + i] = b[o] + sum_k fl(w[o * t_dim + k] * t[r * t_dim + k]), o = mi 6 C + ci C + i,
 *   the sum in k order from -0.0 in float32 (Rust's f32 Sum); out is [6, R * m, C].
 * rotations: (cos, sin) of fl((float) pos * inv_freq[f]) for each token's three axes in order: cs [S, 3 n, 2] with
 *   positions float64 [S, 3] (cosf / sinf of the C library, which Rust's f32::cos and f32::sin call). */
void h3o_adaln_tables(const float* w, const float* b, const float* t_emb, int64_t R, int64_t t_dim, int64_t m, int64_t C,
                      float* out);
void h3o_rotations(const double* positions, int64_t S, const float* inv_freq, int64_t n, float* cs);

/* reference::compare (engine/h3-core/src/reference.rs:84-95): relative L2 error and cosine */
/* token kinds (engine/h3-core/src/layout.rs:21-32) and the layout of one denoiser call (layout.rs:107-176):
 * positions float64 [tokens, 3] and kinds [tokens] (either may be NULL), at most cap rows written; keyframes as three
 * arrays (frame index; video and audio latent frames, -1 for none); returns the number of tokens, or -1 */
enum { H3O_TOK_TEXT = 0, H3O_TOK_COND = 1, H3O_TOK_COND_AUDIO = 2, H3O_TOK_REF_AUDIO = 3, H3O_TOK_AUDIO = 4, H3O_TOK_VIDEO = 5 };
int64_t h3o_layout(int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                   const double* kf_index, const int64_t* kf_video, const int64_t* kf_audio, int64_t n_kf,
                   const int64_t* ref_audio, int64_t n_refs, double* positions, int32_t* kinds, int64_t cap);
void h3o_compare(const float* a, const float* b, int64_t n, double* rel, double* cos);

/* the error of the last failing call (argument checks) */
const char* h3o_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
