// vx_quant.hip — per-(token, group) int8 activation quantizer (QuantAct::quantize_layout, packed.rs:307-436;
// quantize_group_portable, packed.rs:527-535), one wavefront per token row.
//
// Per group: amax = max |x| (a max is exact in any order), s = amax / 127 (1 when amax == 0), inv = 1 / s (IEEE
// division), code = clamp(rint(x * inv), -127, 127) with round-half-to-even, NaN -> 0 as Rust's `as i8`;
// gsum = sum of the codes (exact integer). The codes equal the reference's bit for bit.
//
// Output layout (QuantAct with its transposed scales, packed.rs:291-294): q int8 [n][inp]; scales_t float32
// [ng][n_pad] and gsum_t int32 [ng][n_pad] with n_pad = n rounded up to a multiple of 16, pad tokens zero, so a
// GEMM lane reads the scales of 4 consecutive tokens with one 16-byte load.
#include "vx_internal.h"

namespace vx {

__device__ inline int8_t code_of(float x, float inv) {
    float v = __builtin_rintf(x * inv);
    if (!(v == v)) return 0;
    v = v < -127.0f ? -127.0f : v;
    v = v > 127.0f ? 127.0f : v;
    return (int8_t)(int)v;
}

// Fast path: group = 16 * L with L a power of two up to 64 lanes, or a multiple of 1024. Each lane owns 16
// consecutive values of a 1024-wide chunk; a group is L adjacent lanes (or whole chunks), reduced with xor
// shuffles inside the lane group.
template <int L>
__global__ __launch_bounds__(256) void quantize_fast_kernel(const float *__restrict__ x, int n, int inp, int group,
                                                          int np, int8_t *__restrict__ q, float *__restrict__ st,
                                                          int32_t *__restrict__ gt) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;  // uniform per wavefront
    const float *xr = x + (int64_t)t * inp;
    int8_t *qr = q + (int64_t)t * inp;
    const int ng = inp / group;
    const int chunks_per_group = group >= 1024 ? group / 1024 : 1;
    for (int c0 = 0; c0 < inp; c0 += 1024 * chunks_per_group) {
        // amax over this lane's values of the group (all chunks of the group)
        float m = 0.0f;
        for (int cc = 0; cc < chunks_per_group; cc++) {
            const int base = c0 + cc * 1024 + lane * 16;
            if (base < inp) {
                const float4 *p = (const float4 *)(xr + base);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = p[i];
                    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
                }
            }
        }
#pragma unroll
        for (int o = 1; o < L; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float s = m == 0.0f ? 1.0f : m / 127.0f;
        const float inv = 1.0f / s;
        int sum = 0;
        for (int cc = 0; cc < chunks_per_group; cc++) {
            const int base = c0 + cc * 1024 + lane * 16;
            if (base < inp) {
                const float4 *p = (const float4 *)(xr + base);
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 v = p[i];
                    const int8_t c0_ = code_of(v.x, inv), c1 = code_of(v.y, inv), c2 = code_of(v.z, inv),
                                 c3 = code_of(v.w, inv);
                    sum += (int)c0_ + (int)c1 + (int)c2 + (int)c3;
                    w[i] = (uint32_t)(uint8_t)c0_ | ((uint32_t)(uint8_t)c1 << 8) | ((uint32_t)(uint8_t)c2 << 16) |
                           ((uint32_t)(uint8_t)c3 << 24);
                }
                *(uint4 *)(qr + base) = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (int o = 1; o < L; o <<= 1) sum += __shfl_xor(sum, o, 64);
        // the first lane of each lane group writes its group's scale and code sum
        if ((lane & (L - 1)) == 0) {
            const int base = c0 + lane * 16;
            if (base < inp) {
                const int g = base / group;
                if (g < ng) {
                    st[(int64_t)g * np + t] = s;
                    gt[(int64_t)g * np + t] = sum;
                }
            }
        }
    }
}

// Any group that divides inp: one group at a time across the wavefront.
__global__ __launch_bounds__(256) void quantize_generic_kernel(const float *__restrict__ x, int n, int inp,
                                                             int group, int np, int8_t *__restrict__ q,
                                                             float *__restrict__ st, int32_t *__restrict__ gt) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const float *xr = x + (int64_t)t * inp;
    int8_t *qr = q + (int64_t)t * inp;
    const int ng = inp / group;
    for (int g = 0; g < ng; g++) {
        const float *xg = xr + (int64_t)g * group;
        float m = 0.0f;
        for (int c = lane; c < group; c += 64) m = fmaxf(m, fabsf(xg[c]));
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float s = m == 0.0f ? 1.0f : m / 127.0f;
        const float inv = 1.0f / s;
        int sum = 0;
        for (int c = lane; c < group; c += 64) {
            const int8_t code = code_of(xg[c], inv);
            qr[(int64_t)g * group + c] = code;
            sum += code;
        }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
        if (lane == 0) {
            st[(int64_t)g * np + t] = s;
            gt[(int64_t)g * np + t] = sum;
        }
    }
}

// zero the pad tokens [n, np) of scales_t and gsum_t (ng * (np - n) entries)
__global__ void quantize_pad_kernel(int n, int np, int ng, float *__restrict__ st, int32_t *__restrict__ gt) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int pad = np - n;
    if (i < ng * pad) {
        const int g = i / pad, t = n + i % pad;
        st[(int64_t)g * np + t] = 0.0f;
        gt[(int64_t)g * np + t] = 0;
    }
}

void quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
              hipStream_t stream) {
    require(x && q && scales_t && gsum_t, "x, q, scales_t and gsum_t must not be NULL");
    require(n >= 0 && inp > 0 && group > 0 && inp % group == 0, "inp must be a positive multiple of group");
    require(n * inp < (1ll << 31), "activation block above 2 GiB");
    if (n == 0) return;
    const int np = (int)((n + 15) / 16 * 16), ng = (int)(inp / group);
    const unsigned blocks = (unsigned)((n + 3) / 4);
    const int ni = (int)n, ii = (int)inp, gi = (int)group;
    const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (reinterpret_cast<uintptr_t>(q) % 16 == 0) &&
                         inp % 1024 == 0;
    int L = 0;
    if (aligned) {
        if (group % 1024 == 0)
            L = 64;
        else if (group >= 64 && group <= 1024 && (group & (group - 1)) == 0)
            L = group / 16;
    }
    switch (L) {
        case 4: quantize_fast_kernel<4><<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
        case 8: quantize_fast_kernel<8><<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
        case 16: quantize_fast_kernel<16><<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
        case 32: quantize_fast_kernel<32><<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
        case 64: quantize_fast_kernel<64><<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
        default: quantize_generic_kernel<<<blocks, 256, 0, stream>>>(x, ni, ii, gi, np, q, scales_t, gsum_t); break;
    }
    hip_check(hipGetLastError(), "quantize kernel launch");
    if (np > n) {
        const int cnt = ng * (np - ni);
        quantize_pad_kernel<<<(cnt + 255) / 256, 256, 0, stream>>>(ni, np, ng, scales_t, gsum_t);
        hip_check(hipGetLastError(), "quantize pad kernel launch");
    }
}

}  // namespace vx
