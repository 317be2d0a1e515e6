/* h3hip.h - the C ABI of libh3hip.so: MI355X (gfx950) HIP kernels for the per-token layer work of MiniMax H3.
 *
 * Drop-in for kernels/h3sycl.h of maxfridbe/sycl_minimax_h3. Every function of that header is declared here with the
 * same name, argument list and return convention, so engine/h3-sys (engine/h3-sys/src/lib.rs:215-283, which
 * resolves 48 of these names and refuses a library missing any) loads this library unchanged, found through
 * $H3SYCL_LIB (engine/h3-sys/src/lib.rs:181-193). Functions that have no HIP implementation here (the convolutions,
 * the upscaler's and the audio decoder's ops, k-quant expansion) return -1 with a message naming them.
 *
 * Conventions, as kernels/h3sycl.h:1-9:
 *  - every data pointer is device memory of the context's GPU;
 *  - kernels are asynchronous and run in call order on the context's one HIP stream; h3s_read, h3s_write and
 *    h3s_wait are the points that wait;
 *  - int functions return 0, or -1 with the reason in h3s_last_error() (per thread); pointer functions return NULL
 *    on failure, same; arguments are checked before any work is queued; empty shapes return 0 and do nothing.
 *
 * Element types: H3S_F32 = 0, H3S_F16 = 1, H3S_BF16 = 2 (kernels/h3sycl.h:20).
 *
 * Layout preconditions of the vectorized kernels (16-byte loads, no scalar fallback): rows of C features must be
 * whole 16-byte vectors (C a multiple of 8 for 16-bit types, of 4 for float32) and every tensor 16-byte aligned
 * (h3s_alloc memory is). A call that breaks them returns -1 with the reason.
 */
#ifndef H3HIP_H
#define H3HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types of floating-point tensors (kernels/h3sycl.h:20) */
enum { H3S_F32 = 0, H3S_F16 = 1, H3S_BF16 = 2 };

/* block rotations before quantization (additions: kernels/h3sycl.h:74-83 defines only the regular one) */
enum { H3S_ROT_NONE = 0, H3S_ROT_REGULAR = 1, H3S_ROT_SYLVESTER = 2 };
/* pointwise activations of the fused chains (additions) */
enum { H3S_ACT_NONE = 0, H3S_ACT_GELU_TANH = 1, H3S_ACT_SILU = 2 };
/* row norms of the fused modulate chain (additions) */
enum { H3S_NORM_RMS = 0, H3S_NORM_LAYER = 1 };

/* replaces kernels/h3sycl.h:22 */
const char* h3s_last_error(void);

/* ---- context ---------------------------------------------------------------------------------------------- */

/* A context on GPU 0 with its own stream. Replaces kernels/h3sycl.h:27. */
void* h3s_open(void);
/* The GPUs HIP sees; name, memory size and PCI address ("0000:0b:00.0"). Replaces kernels/h3sycl.h:30-31. */
int h3s_gpu_count(void);
int h3s_gpu_info(int index, char* name, int name_len, uint64_t* mem_bytes, char* pci, int pci_len);
/* A context on GPU `index`. Replaces kernels/h3sycl.h:32. */
void* h3s_open_gpu(int index);
/* A context around an existing hipStream_t (PyTorch: torch.cuda.current_stream().cuda_stream) on the current
 * device; the stream is used, not owned. Replaces kernels/h3sycl.h:35 (which takes a sycl::queue*). */
void* h3s_create(void* hip_stream);
/* Waits for the stream, frees the scratch and everything still allocated with h3s_alloc. Replaces h3sycl.h:37. */
void h3s_destroy(void* ctx);
/* replaces kernels/h3sycl.h:39 */
const char* h3s_device_name(void* ctx);

/* ---- device memory: replaces kernels/h3sycl.h:43-70 ---------------------------------------------------------- */

/* Counted allocations: one that would pass the cap (0.94 of the card; H3S_MEM_FRACTION overrides, clamped to
 * [0.05, 0.97]) is refused with an error. The library's own scratch counts against the same cap. */
void* h3s_alloc(void* ctx, uint64_t bytes);
void h3s_free(void* ctx, void* p); /* waits for the stream first */
uint64_t h3s_mem_used(void* ctx);
uint64_t h3s_mem_cap(void* ctx);
uint64_t h3s_mem_free(void* ctx);
/* host <-> device, both wait */
int h3s_write(void* ctx, void* dst, const void* src_host, uint64_t bytes);
int h3s_read(void* ctx, void* dst_host, const void* src, uint64_t bytes);
/* device to device, queued */
int h3s_copy(void* ctx, void* dst, const void* src, uint64_t bytes);
int h3s_wait(void* ctx);
/* pinned host memory and uploads on a second stream beside the kernels */
void* h3s_alloc_host(void* ctx, uint64_t bytes);
void h3s_free_host(void* ctx, void* p);
int h3s_upload(void* ctx, void* dst, const void* src_pinned, uint64_t bytes);
int h3s_upload_wait(void* ctx);

/* ---- the reference's kernels -------------------------------------------------------------------------------- */

/* int8 linear with activations quantized on the fly (kernels/h3sycl.h:74-85):
 *   x_rot = x . H per group (regular Hadamard, group a power of 4 at most 256, or 0 for none)
 *   s_r = max(max|x_rot[r]| / 127, 1e-30); q = clamp(rint(x_rot / s_r), -128, 127)
 *   out = acc * fl(s_r * wscale[0]) (one scale) or (acc * s_r) * wscale[n] (N scales), + bias[n]
 * The GEMM runs on i8 MFMA with the rescale in its epilogue. */
int h3s_int8_linear(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                    const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt, int group);

/* Float linear layers (kernels/h3sycl.h:89-95): h3s_linear out = x w^T + bias, h3s_linear_acc out += x w^T + bias,
 * h3s_scale_rows x[r] *= s[r]. Float32 accumulation on the context's stream: bfloat16 and half operands with K a
 * multiple of 32, more than 128 outputs a row and 16-byte aligned rows on the library's own matrix-core kernel, every
 * other call on rocBLAS; the bias and the old output are added in float32 and rounded once to the output type. */
int h3s_linear_acc(void* ctx, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N, const float* bias, void* out);
int h3s_scale_rows(void* ctx, void* x, int dt, int64_t M, int64_t C, const float* s);
int h3s_linear(void* ctx, const void* x, int dt, int64_t M, int64_t K, const void* w, int64_t N, const float* bias,
               void* out, int out_dt);

/* Causal attention with grouped heads (kernels/h3sycl.h:104-108): Hq query heads over Hkv key/value heads, rows of
 * q at stride qs and of k, v at stride kvs; the 16-bit form. Any head size up to 256 (zero-padded to 64, 128 or 256
 * features inside, the output stored at D). */
int h3s_attention_causal(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t L, int64_t Hq, int64_t Hkv, int64_t D,
                         int64_t qs, int64_t kvs, void* out);
/* Not implemented here (text encoder, upscalers, audio): -1. Replace kernels/h3sycl.h:106-158. */
int h3s_dequant(void* ctx, const void* src, int qtype, int64_t n, void* out, int out_dt);
int h3s_conv3d(void* ctx, const void* x, int dt, int64_t T, int64_t H, int64_t W, int64_t Ci, const void* w, int64_t Co, int64_t k,
               const float* bias, void* out);
int h3s_group_norm_silu(void* ctx, const void* x, int dt, int64_t F, int64_t N, int64_t C, int64_t G, const float* weight, const float* bias,
                        float eps, const float* scale, const float* shift, void* out);
int h3s_pad3d(void* ctx, const void* x, int dt, int64_t T, int64_t H, int64_t W, int64_t C, int64_t front, int64_t top, int64_t bottom,
              int64_t left, int64_t right, void* out);
int h3s_conv2d(void* ctx, const void* x, int dt, int64_t N, int64_t H, int64_t W, int64_t Ci, const void* w, int64_t Co, int64_t k,
               const float* bias, void* out);
int h3s_prelu(void* ctx, void* x, int dt, int64_t M, int64_t C, const float* alpha);
int h3s_pixel_shuffle_add(void* ctx, const void* x, int dt, int64_t N, int64_t H, int64_t W, int64_t C, int64_t r,
                          const void* base, void* out);
int h3s_resize_area(void* ctx, const void* x, int dt, int64_t N, int64_t Hi, int64_t Wi, int64_t C, int64_t Ho, int64_t Wo,
                    float* out);
int h3s_conv3d_ex(void* ctx, const void* x, int dt, int64_t T, int64_t H, int64_t W, int64_t Ci, const void* w, int64_t Co,
                  int64_t kt, int64_t kh, int64_t kw, int64_t st, int64_t sh, int64_t sw, const float* bias, void* out);
int h3s_temporal_dwconv(void* ctx, const void* x, int dt, int64_t T, int64_t P, int64_t C, const float* w, int64_t K,
                        const float* bias, void* out);
int h3s_trilinear(void* ctx, const void* x, int dt, int64_t T, int64_t H, int64_t W, int64_t C, int64_t To, int64_t Ho, int64_t Wo,
                  void* out);
int h3s_conv1d(void* ctx, const float* x, int64_t B, int64_t Ci, int64_t L, const float* w, int64_t Co, int64_t K,
               const float* bias, int64_t stride, int64_t dil, int64_t pad, float* out, int64_t Lo);
int h3s_conv_transpose1d(void* ctx, const float* x, int64_t B, int64_t Ci, int64_t L, const float* w, int64_t Co, int64_t K,
                         const float* bias, int64_t stride, int64_t pad, float* out, int64_t Lo);
int h3s_aa_snake(void* ctx, const float* x, int64_t B, int64_t C, int64_t L, const float* log_alpha, const float* log_beta,
                 const float* up, const float* down, float* out);
int h3s_scale(void* ctx, float* x, int64_t n, float s);
int h3s_snake(void* ctx, const float* x, int64_t B, int64_t C, int64_t L, const float* alpha, float* out);

/* Layer norm per row: (x - mean) / sqrt(var + eps) * weight + bias, weight and bias float32 [C] or NULL.
 * Replaces kernels/h3sycl.h:159-161. */
int h3s_layer_norm(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, const float* bias, float eps,
                   void* out, int out_dt);
/* RMS norm per row, then out = n * (1 + scale[rows[r]]) + shift[rows[r]] when rows, scale and shift are all given.
 * x, out [M, C]; weight float32 [C]; scale, shift float32 [R, C]. out may be x. Replaces kernels/h3sycl.h:162-163. */
int h3s_rms_norm_mod(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps,
                     const int32_t* rows, const float* scale, const float* shift, void* out, int out_dt);
/* Per-head RMS norm, then the rotary rotation of pairs (i, rot_dim/2 + i) by cs float32 [M, rot_dim/2, 2], in place;
 * row m at element m * stride. Replaces kernels/h3sycl.h:173-174. Any even rot_dim <= D that leaves an even
 * remainder, as the reference; D and the stride must be whole 16-byte vectors (8 elements of a 16-bit type, 4 of
 * float32), and a head at most 64 16-byte slots. */
int h3s_rms_rope(void* ctx, void* x, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride, const float* weight,
                 float eps, const float* cs, int rot_dim);
/* out[r, i] = silu(x[r, i]) * x[r, C + i]. Replaces kernels/h3sycl.h:178. */
int h3s_swiglu(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, void* out, int out_dt);
/* x[r] += other[r] * gate[rows[r]] in place; gate NULL: a plain add. Replaces kernels/h3sycl.h:182-183. */
int h3s_gate_add(void* ctx, void* x, int x_dt, int64_t M, int64_t C, const void* other, int other_dt,
                 const int32_t* rows, const float* gate);

/* Attention over S tokens of H heads of D (any head size up to 256), rows at element stride `stride`, out [S, H D]
 * (h3s_attention), and B independent sequences of S tokens each (h3s_attention_batch). The reference's choice of form: the int8
 * (SageAttention) form from H3S_SAGE_MIN_S tokens (8192) on for heads of 64 or 128 features unless H3S_ATTN=onednn
 * (kernels/h3sycl.cpp:1706), the 16-bit form otherwise.
 * Replace kernels/h3sycl.h:190-200. */
int h3s_attention(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t S, int64_t H, int64_t D,
                  int64_t stride, void* out, int out_dt);
int h3s_attention_batch(void* ctx, const void* q, const void* k, const void* v, int dt, int64_t B, int64_t S, int64_t H,
                        int64_t D, int64_t stride, void* out, int out_dt);

/* ---- additions: fused entry points (no counterpart in kernels/h3sycl.h; the h3-sys loader ignores them) ------ */

/* The context's HIP stream (hipStream_t), for callers that time or order work around the library's kernels. */
void* h3s_stream(void* ctx);

/* rms_norm_mod then int8_linear's quantizer, in one pass over x (the pair at engine/h3-core/src/dit.rs:340-342):
 *   n = round_to_h_dt(x * inv_rms * weight [* (1 + scale[t]) + shift[t]])       (the bf16 scratch h of the reference)
 *   y = n . H per group when rot != NONE (REGULAR: g = 4^k; SYLVESTER: g = 2^k, H2^(x)k / sqrt(g))
 *   s[r] = max(max|y| / 127, 1e-30); q = clamp(rint(y / s[r]), -128, 127)
 * weight float32 [C] or NULL (1); scale/shift tables [R, C] in tab_dt (F32 or BF16) or NULL (no modulation);
 * rows int32 [M] or NULL (every token uses table row 0). q int8 [M, C], s float32 [M]: the pure activation scale. */
int h3s_norm_quant(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, const float* weight, float eps,
                   const int32_t* rows, const void* scale, const void* shift, int tab_dt, int h_dt, int rot, int group,
                   int8_t* q, float* s);

/* h3s_swiglu then int8_linear's quantizer, in one pass over x (the MLP's act scratch and fc2's quantizer at
 * engine/h3-core/src/dit.rs:363-364; kernels/h3sycl.cpp:1378-1419 and 404-474):
 *   a = round_to_h_dt(silu(g) * u) with g = x[r, i], u = x[r, C + i]            (x rows of 2C, as h3s_swiglu)
 *   then rotation and quantization of a as in h3s_norm_quant (rot, group; h3s_int8_linear's group is REGULAR).
 * q int8 [M, C], s float32 [M]: the inputs of h3s_int8_gemm_dequant for fc2. */
int h3s_swiglu_quant(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, int h_dt, int rot, int group, int8_t* q,
                     float* s);

/* h3s_int8_linear's quantizer on its own, the first of its two passes (kernels/h3sycl.cpp:404-474, 521-575):
 * x [M, K] in x_dt, rotated per group of `group` features by the regular Hadamard (0: no rotation), then
 * s[r] = max(max|y| / 127, 1e-30), q = rint(y / s[r]). q int8 [M, K], s float32 [M]: the inputs of h3s_int8_gemm_dequant. */
int h3s_int8_quantize(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, int group, int8_t* q, float* s);

/* What a sampler step fixes for every block, on the device instead of the reference's host loops:
 * h3s_adaln_tables (engine/h3-core/src/dit.rs:155-174, Block::tables): the six AdaLN tables of one block for R timestep
 *   embeddings t_emb [R, t_dim]; w [6 m C, t_dim], b [6 m C] (the block's adaln_proj), all float32;
 *   out [6, R * m, C]: table ci (shift, scale, gate of the attention half, then of the MLP half) at out + ci R m C, row
 *   r m + mi, value b[o] + sum_k w[o, k] t[r, k] with o = mi 6 C + ci C + i, summed in k order in float32.
 * h3s_rotations (engine/h3-core/src/dit.rs:188-203, rotations): cs [S, 3 n, 2] float32, the (cos, sin) of
 *   fl((float) positions[s, a] * inv_freq[f]) for the axes a = 0, 1, 2 in turn; positions float64 [S, 3]. */
int h3s_adaln_tables(void* ctx, const float* w, const float* b, const float* t_emb, int64_t R, int64_t t_dim, int64_t m,
                     int64_t C, float* out);
int h3s_rotations(void* ctx, const double* positions, int64_t S, const float* inv_freq, int64_t n, float* cs);

/* out = res + gate * act(norm(x) * (1 + scale) + shift), in one pass; norm RMS (x * inv_rms * weight) or LAYER
 * ((x - mean) * inv_std * weight + bias); weight, bias float32 [C] or NULL; tables [R, C] in tab_dt with rows as in
 * h3s_norm_quant; gate NULL: 1; res NULL: none. Everything in float32, one rounding to out_dt at the end. */
int h3s_norm_mod_act_gate(void* ctx, const void* x, int x_dt, int64_t M, int64_t C, int norm, const float* weight,
                          const float* bias, float eps, const int32_t* rows, const void* scale, const void* shift,
                          const void* gate, int tab_dt, int act, const void* res, int res_dt, void* out, int out_dt);

/* h3s_rms_rope on q (weight wq) and k (weight wk) in one launch, with one read of cs per token (the pair at
 * engine/h3-core/src/dit.rs:347-348). q and k share M, H, D, stride and x_dt; they may sit in one qkv buffer. */
int h3s_qk_rms_rope(void* ctx, void* q, void* k, int x_dt, int64_t M, int64_t H, int64_t D, int64_t stride,
                    const float* wq, const float* wk, float eps, const float* cs, int rot_dim);

/* The int8 GEMM of h3s_int8_linear from already quantized activations, with an activation in the epilogue:
 *   out[m, n] = act(acc * fl(s[m] * wscale[0]) + bias[n])   (n_wscale = 1)
 *   out[m, n] = act((acc * s[m]) * wscale[n] + bias[n])      (n_wscale = N)
 * q int8 [M, K]; s float32 [M]; w int8 [N, K]; bias float32 [N] or NULL; out [M, N] in out_dt. K a multiple of 64. */
int h3s_int8_gemm_dequant(void* ctx, const int8_t* q, const float* s, int64_t M, int64_t K, const int8_t* w, int64_t N,
                          const float* wscale, int64_t n_wscale, const float* bias, int act, void* out, int out_dt);

/* The token layout of one denoiser call (engine/h3-core/src/layout.rs:107-176, Layout::new), owned by the library.
 * The sequence is [text | keyframe conditioning | reference audio | audio | video]; a token's kind is one of: */
enum { H3S_TOK_TEXT = 0, H3S_TOK_COND = 1, H3S_TOK_COND_AUDIO = 2, H3S_TOK_REF_AUDIO = 3, H3S_TOK_AUDIO = 4, H3S_TOK_VIDEO = 5 };
/* A keyframe to condition on (layout.rs:45-52): its place on the target timeline in pixel frames, and the latent
 * frames of video and of audio it brings (-1: none). */
typedef struct {
    double frame_index;
    int64_t video_latent_t;
    int64_t audio_latent_t;
} h3s_keyframe;
/* h3s_layout_plan (host only, no device): the segments of the sequence in row order - seg_start, seg_stop (rows) and
 *   seg_kind, at most seg_cap of each written, any of them NULL - for a text of text_len tokens, a video latent
 *   [latent_t, latent_h, latent_w] (even height and width; a token is 2 x 2 latent pixels), audio_t audio latent
 *   frames (two rows each, one per stereo channel), n_keyframes keyframes and n_refs reference voices of ref_audio[i]
 *   audio latent frames. Returns the number of segments (the last one's stop is the token count), or -1.
 * h3s_layout: for the same request, each token's position (time, height, width) into positions float64 [tokens, 3],
 *   with the reference's float64 arithmetic, and with rows not NULL its AdaLN table row rows[t] = row_of_kind[kind]
 *   (row_of_kind: 6 host int32, the row each kind reads at the step). tokens must be the layout's token count. */
int64_t h3s_layout_plan(int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                        const h3s_keyframe* keyframes, int64_t n_keyframes, const int64_t* ref_audio, int64_t n_refs,
                        int64_t* seg_start, int64_t* seg_stop, int32_t* seg_kind, int64_t seg_cap);
int h3s_layout(void* ctx, int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
               const h3s_keyframe* keyframes, int64_t n_keyframes, const int64_t* ref_audio, int64_t n_refs,
               const int32_t* row_of_kind, double* positions, int32_t* rows, int64_t tokens);

/* h3s_int8_linear without any allocation: no counterpart in the reference. For callers that cannot allocate device
 * memory - code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. Same arguments and
 * results as h3s_int8_linear; the quantized rows go into a fixed device array of the library (64 MiB of codes and
 * 65536 row scales, held on each GPU the library runs on until the process ends) instead of the context's scratch.
 * Any M (rows go through in chunks that fit the array); K at most 65536, else -1 with the reason. Calls on one GPU
 * share its array: calls that overlap on one GPU (two streams or two contexts at once) race. The array (64.25 MiB a
 * GPU) is part of the library's code object, not of a context: it is outside the H3S_MEM_FRACTION cap and is not
 * counted by h3s_mem_used. */
int h3s_int8_linear_noalloc(void* ctx, const void* x, int x_dt, int64_t M, int64_t K, const int8_t* w, int64_t N,
                            const float* wscale, int64_t n_wscale, const float* bias, void* out, int out_dt, int group);
/* How many device and host allocations, events, streams and library handles libh3hip has made in this process, counted
 * as they are attempted. No counterpart in the reference: a diagnostic, for tests and callers that must show a call
 * path allocates nothing (h3s_int8_linear_noalloc leaves it unchanged). */
uint64_t h3s_alloc_count(void);

#ifdef __cplusplus
}
#endif
#endif
