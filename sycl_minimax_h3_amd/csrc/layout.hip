// layout.hip - the token layout of one denoiser call (engine/h3-core/src/layout.rs:107-176): h3s_layout_plan, the
// segments of the sequence [text | keyframe conditioning | reference audio | audio | video] on the host, and
// h3s_layout, each token's position (time, height, width) and AdaLN table row on the device.
//
// The plan is a list of spans, each a run of rows of one kind laid out in one of three forms:
//   text   row j of the span sits at (j, 0, 0);
//   audio  two stereo channels one after the other, each `frames` rows at (origin + f, 0, w) with w the first or
//          the last width coordinate of the video frame;
//   video  `frames` latent frames of nh x nw patches each, frame k at time t_k, patch (a, b) at (H_a, W_b).
// A device thread per token finds its span and computes its three coordinates in closed form from the span's
// numbers, with the same float64 operations in the same order as the reference: the axis coordinate
// (i * (ratio / n) + (1 - ratio) / 2) * 32 and the frame times t_{k+1} = t_k + (5/3) x (1, 4, 4, 4, 4)[k % 5]
// summed from the span's origin, so every position has the reference's bits.
#include <cmath>
#include <vector>

#include "common.h"

namespace h3 {

constexpr int kMaxSpans = 24;                   // text, audio, video, and up to 9 keyframes with both parts or refs
enum SpanForm : int32_t { FORM_TEXT = 0, FORM_AUDIO = 1, FORM_VIDEO = 2 };

struct Span {
    int64_t start, rows, frames;                // frames: audio frames a channel, or video frames
    double origin;                              // the time of the span's first row
    int32_t kind, form;
};

struct LayoutPlan {
    int32_t n = 0;
    Span spans[kMaxSpans];
    int64_t nh = 0, nw = 0;                     // patches along the height and the width of a video frame
    double hq = 0, hc = 0, wq = 0, wc = 0;      // axis coordinate i: (i * q + c) * 32
    int32_t row_of_kind[6] = {0, 0, 0, 0, 0, 0};
};

// (i * (ratio / n) + (1 - ratio) / 2) * 32 (layout.rs:88-93)
__host__ __device__ __forceinline__ double axis_at(int64_t i, double q, double c) { return ((double) i * q + c) * 32.0; }

// the plan of a call; false with the reason as this thread's error
static bool make_plan(const char* fn, int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                      const h3s_keyframe* keyframes, int64_t n_keyframes, const int64_t* ref_audio, int64_t n_refs,
                      LayoutPlan& P) {
    if (latent_h <= 0 || latent_w <= 0 || latent_h % 2 || latent_w % 2)
        return fail(std::string(fn) + ": the video latent's height and width must be even and positive, got " +
                    std::to_string(latent_h) + " x " + std::to_string(latent_w)) == 0;
    if (text_len < 0 || latent_t < 0 || audio_t < 0 || n_keyframes < 0 || n_refs < 0 || (n_keyframes && !keyframes) ||
        (n_refs && !ref_audio))
        return fail(std::string(fn) + ": negative counts, or keyframes / references missing") == 0;
    const double sqrt_area = std::sqrt((double) (latent_h * latent_w));
    const double rh = (double) latent_h / sqrt_area, rw = (double) latent_w / sqrt_area;
    P.nh = latent_h / 2;
    P.nw = latent_w / 2;
    P.hq = rh / (double) P.nh;
    P.hc = (1.0 - rh) / 2.0;
    P.wq = rw / (double) P.nw;
    P.wc = (1.0 - rw) / 2.0;
    int64_t row = 0;
    auto add = [&](int32_t kind, int32_t form, int64_t frames, double origin) -> bool {
        if (P.n == kMaxSpans) return false;
        const int64_t rows = form == FORM_TEXT ? frames : form == FORM_AUDIO ? 2 * frames : frames * P.nh * P.nw;
        P.spans[P.n++] = Span{row, rows, frames, origin, kind, form};
        row += rows;
        return true;
    };
    // the references sit right after the text on the time axis, the targets after them (layout.rs:146-147)
    double refs_span = 0.0;
    for (int64_t i = 0; i < n_refs; ++i) {
        if (ref_audio[i] < 0) return fail(std::string(fn) + ": a negative reference length") == 0;
        refs_span += (double) ref_audio[i];
    }
    const double cursor = (double) text_len + refs_span;
    bool ok = add(H3S_TOK_TEXT, FORM_TEXT, text_len, 0.0);
    for (int64_t i = 0; i < n_keyframes && ok; ++i) {
        const h3s_keyframe& kf = keyframes[i];
        const double at = cursor + (5.0 / 3.0) * kf.frame_index;
        if (kf.video_latent_t >= 0) ok = ok && add(H3S_TOK_COND, FORM_VIDEO, kf.video_latent_t, at);
        if (kf.audio_latent_t >= 0) ok = ok && add(H3S_TOK_COND_AUDIO, FORM_AUDIO, kf.audio_latent_t, at);
    }
    double rc = (double) text_len;
    for (int64_t i = 0; i < n_refs && ok; ++i) {
        if (ref_audio[i] > 0) ok = add(H3S_TOK_REF_AUDIO, FORM_AUDIO, ref_audio[i], rc);
        rc += (double) ref_audio[i];
    }
    ok = ok && add(H3S_TOK_AUDIO, FORM_AUDIO, audio_t, cursor);
    ok = ok && add(H3S_TOK_VIDEO, FORM_VIDEO, latent_t, cursor);
    if (!ok) return fail(std::string(fn) + ": more than " + std::to_string(kMaxSpans) + " segments") == 0;
    return true;
}

__global__ __launch_bounds__(256) void layout_kernel(LayoutPlan P, double* __restrict__ pos, int32_t* __restrict__ rows,
                                                     int64_t tokens) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= tokens) return;
    int s = 0;
    while (s + 1 < P.n && i >= P.spans[s + 1].start) ++s;    // spans in row order; an empty span shares its start
    const Span sp = P.spans[s];
    const int64_t j = i - sp.start;
    double t = 0.0, h = 0.0, w = 0.0;
    if (sp.form == FORM_TEXT) {
        t = (double) j;
    } else if (sp.form == FORM_AUDIO) {
        const int64_t ch = j / sp.frames, f = j - ch * sp.frames;   // channel-major (layout.rs:133-140)
        t = sp.origin + (double) f;
        w = ch ? axis_at(P.nw - 1, P.wq, P.wc) : axis_at(0, P.wq, P.wc);
    } else {
        const int64_t per = P.nh * P.nw, k = j / per, r = j - k * per;
        t = sp.origin;
        for (int64_t f = 0; f < k; ++f) t += (5.0 / 3.0) * (f % 5 == 0 ? 1.0 : 4.0);   // layout.rs:96-105
        h = axis_at(r / P.nw, P.hq, P.hc);
        w = axis_at(r % P.nw, P.wq, P.wc);
    }
    pos[3 * i] = t;
    pos[3 * i + 1] = h;
    pos[3 * i + 2] = w;
    if (rows) rows[i] = P.row_of_kind[sp.kind];
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int64_t h3s_layout_plan(int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                                   const h3s_keyframe* keyframes, int64_t n_keyframes, const int64_t* ref_audio, int64_t n_refs,
                                   int64_t* seg_start, int64_t* seg_stop, int32_t* seg_kind, int64_t seg_cap) try {
    LayoutPlan P;
    if (!make_plan("h3s_layout_plan", text_len, latent_t, latent_h, latent_w, audio_t, keyframes, n_keyframes, ref_audio,
                   n_refs, P))
        return -1;
    for (int32_t s = 0; s < P.n && s < seg_cap; ++s) {
        if (seg_start) seg_start[s] = P.spans[s].start;
        if (seg_stop) seg_stop[s] = P.spans[s].start + P.spans[s].rows;
        if (seg_kind) seg_kind[s] = P.spans[s].kind;
    }
    return P.n;
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_layout(void* ctx, int64_t text_len, int64_t latent_t, int64_t latent_h, int64_t latent_w, int64_t audio_t,
                          const h3s_keyframe* keyframes, int64_t n_keyframes, const int64_t* ref_audio, int64_t n_refs,
                          const int32_t* row_of_kind, double* positions, int32_t* rows, int64_t tokens) try {
    const char* fn = "h3s_layout";
    LayoutPlan P;
    if (!make_plan(fn, text_len, latent_t, latent_h, latent_w, audio_t, keyframes, n_keyframes, ref_audio, n_refs, P)) return -1;
    const int64_t total = P.spans[P.n - 1].start + P.spans[P.n - 1].rows;
    if (tokens != total)
        return fail(std::string(fn) + ": the layout has " + std::to_string(total) + " tokens, the buffers " + std::to_string(tokens));
    if (!positions) return fail(std::string(fn) + ": positions are required");
    if (rows && !row_of_kind) return fail(std::string(fn) + ": table rows need the row of each kind");
    if (row_of_kind)
        for (int k = 0; k < 6; ++k) P.row_of_kind[k] = row_of_kind[k];
    if (total == 0) return 0;
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    layout_kernel<<<(unsigned) ((total + 255) / 256), 256, 0, c->stream>>>(P, positions, rows, total);
    return launched(fn);
} catch (const std::exception& e) { return fail(e.what()); }
