// vx_quant.hip — per-(token, group) int8 activation quantizer (QuantAct::quantize_layout, packed.rs:307-436;
// quantize_group_portable, packed.rs:527-535), one wavefront per token row.
//
// Per group: amax = max |x| (a max is exact in any order), s = amax / 127 (1 when amax == 0), inv = 1 / s (IEEE
// division), code = clamp(rint(x * inv), -127, 127) with round-half-to-even, NaN -> 0 as Rust's `as i8`.
// gsum = sum of the codes (exact integer). The codes equal the reference's bit for bit.
#include "vx_internal.h"

namespace vx {

__device__ inline float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ inline int wave_sum(int v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__global__ __launch_bounds__(256) void quantize_kernel(const float *__restrict__ x, int64_t n, int64_t inp,
                                                      int64_t group, int8_t *__restrict__ q,
                                                      float *__restrict__ scales, int32_t *__restrict__ gsum) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;  // uniform per wavefront
    const float *xr = x + t * inp;
    int8_t *qr = q + t * inp;
    const int64_t ng = inp / group;
    for (int64_t g = 0; g < ng; g++) {
        const float *xg = xr + g * group;
        float m = 0.0f;
        for (int64_t c = lane; c < group; c += 64) m = fmaxf(m, fabsf(xg[c]));
        m = wave_max(m);
        const float s = m == 0.0f ? 1.0f : m / 127.0f;
        const float inv = 1.0f / s;
        int sum = 0;
        for (int64_t c = lane; c < group; c += 64) {
            float v = __builtin_rintf(xg[c] * inv);
            int code = 0;
            if (v == v) {
                v = v < -127.0f ? -127.0f : v;
                v = v > 127.0f ? 127.0f : v;
                code = (int)v;
            }
            qr[g * group + c] = (int8_t)code;
            sum += code;
        }
        sum = wave_sum(sum);
        if (lane == 0) {
            scales[t * ng + g] = s;
            if (gsum) gsum[t * ng + g] = sum;
        }
    }
}

void quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales, int32_t *gsum,
              hipStream_t stream) {
    require(x && q && scales, "x, q and scales must not be NULL");
    require(n >= 0 && inp > 0 && group > 0 && inp % group == 0, "inp must be a positive multiple of group");
    if (n == 0) return;
    int64_t blocks = (n + 3) / 4;
    require(blocks < (1ll << 31), "too many tokens");
    quantize_kernel<<<(unsigned)blocks, 256, 0, stream>>>(x, n, inp, group, q, scales, gsum);
    hip_check(hipGetLastError(), "quantize_kernel launch");
}

}  // namespace vx
