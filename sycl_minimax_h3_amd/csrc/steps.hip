// steps.hip - what a sampler step fixes for every block, on the device (engine/h3-core/src/dit.rs:155-203, a host
// loop in the reference): h3s_adaln_tables (the six AdaLN tables of a block from the timestep embeddings) and
// h3s_rotations (the (cos, sin) table of every token's position).
#include <cmath>

#include "common.h"

namespace h3 {

// out[ci][(r m + mi) C + i] = b[o] + sum_k fl(w[o, k] t[r, k]), o = mi 6 C + ci C + i: the sum in k order from -0.0
// in float32 (dit.rs:163-170, Rust's f32 Sum), one multiply and one add a term (no fused multiply-add). A wavefront
// takes 64 consecutive o of one timestep row r; their w rows go through LDS 64 columns at a time (coalesced loads),
// and each lane runs its own sum.
__global__ __launch_bounds__(64) void adaln_tables_kernel(const float* __restrict__ w, const float* __restrict__ b,
                                                          const float* __restrict__ t, int64_t R, int64_t td, int64_t m,
                                                          int64_t C, float* __restrict__ out) {
    __shared__ float tile[64][65];
    __shared__ float tk[64];
    const int lane = threadIdx.x;
    const int64_t nout = 6 * m * C, o0 = (int64_t) blockIdx.x * 64, r = blockIdx.y;
    const int64_t o = o0 + lane;
    float sum = -0.0f;
    for (int64_t k0 = 0; k0 < td; k0 += 64) {
        const int kn = td - k0 < 64 ? (int) (td - k0) : 64;
        for (int row = 0; row < 64; ++row) {
            const int64_t oo = o0 + row;
            tile[row][lane] = oo < nout && lane < kn ? w[oo * td + k0 + lane] : 0.0f;
        }
        tk[lane] = lane < kn ? t[r * td + k0 + lane] : 0.0f;
        __syncthreads();
        for (int k = 0; k < kn; ++k) sum = sum + tile[lane][k] * tk[k];
        __syncthreads();
    }
    if (o < nout) {
        const int64_t mi = o / (6 * C), ci = (o / C) % 6, i = o % C;
        out[ci * R * m * C + (r * m + mi) * C + i] = b[o] + sum;
    }
}

// cs[s][a n + f] = (cos x, sin x), x = fl((float) pos[s, a] * inv_freq[f]) (dit.rs:190-203); cos and sin of the float
// argument evaluated in float64 and rounded once, so they are the correctly rounded float32 values
__global__ __launch_bounds__(256) void rotations_kernel(const double* __restrict__ pos, int64_t S, const float* __restrict__ inv,
                                                        int64_t n, float* __restrict__ cs) {
    const int64_t id = (int64_t) blockIdx.x * 256 + threadIdx.x, total = S * 3 * n;
    if (id >= total) return;
    const int64_t f = id % n, sa = id / n;                  // sa = s * 3 + a
    const float x = (float) pos[sa] * inv[f];
    cs[2 * id] = (float) cos((double) x);
    cs[2 * id + 1] = (float) sin((double) x);
}

}  // namespace h3

using namespace h3;

H3S_EXPORT int h3s_adaln_tables(void* ctx, const float* w, const float* b, const float* t_emb, int64_t R, int64_t t_dim,
                                int64_t m, int64_t C, float* out) try {
    const char* fn = "h3s_adaln_tables";
    if (R <= 0 || t_dim <= 0 || m <= 0 || C <= 0) return 0;
    if (!w || !b || !t_emb || !out) return fail(std::string(fn) + ": w, b, t_emb and out are required");
    if (R > 65535) return fail(std::string(fn) + ": at most 65535 timestep rows");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const int64_t nout = 6 * m * C;
    adaln_tables_kernel<<<dim3((unsigned) ((nout + 63) / 64), (unsigned) R), 64, 0, c->stream>>>(w, b, t_emb, R, t_dim, m, C, out);
    return launched(fn);
} catch (const std::exception& e) { return fail(e.what()); }

H3S_EXPORT int h3s_rotations(void* ctx, const double* positions, int64_t S, const float* inv_freq, int64_t n, float* cs) try {
    const char* fn = "h3s_rotations";
    if (S <= 0 || n <= 0) return 0;
    if (!positions || !inv_freq || !cs) return fail(std::string(fn) + ": positions, inv_freq and cs are required");
    Ctx* c = ctx_of(ctx, fn);
    if (!c) return -1;
    const int64_t total = S * 3 * n;
    rotations_kernel<<<(unsigned) ((total + 255) / 256), 256, 0, c->stream>>>(positions, S, inv_freq, n, cs);
    return launched(fn);
} catch (const std::exception& e) { return fail(e.what()); }
