// vx_quant.hip — per-(token, group) int8 activation quantizer (QuantAct::quantize_layout, packed.rs:307-436;
// quantize_group_portable, packed.rs:527-535), one wavefront per token row.
//
// Per group: amax = max |x| (a max is exact in any order), s = amax / 127 (1 when amax == 0), inv = 1 / s (IEEE
// division), code = clamp(rint(x * inv), -127, 127) with round-half-to-even, NaN -> 0 as Rust's `as i8`;
// gsum = sum of the codes (exact integer). The codes equal the reference's bit for bit.
//
// The LN variants (prepare_normed, ternary_linear.rs:132-155) quantize LayerNorm(x) instead of x: the row's mean and
// variance are taken in the reference's order (row_mean_var_portable, tensor.rs:331-363: eight running sums over
// 8-column steps, one per lane of lanes 0-7, combined as hsum4 of the lane pairs, then the tail in order; squares
// by fma), inv = 1 / sqrt(var + 1e-5), and each element is ((x - mean) * inv) * g + b (tensor.rs:712-719) as it is
// quantized, so the normalized row never goes to memory.
//
// Output layout (QuantAct with its transposed scales, packed.rs:291-294): q int8 [n][inp]; scales_t float32
// [ng][n_pad] and gsum_t int32 [ng][n_pad] with n_pad = n rounded up to a multiple of 16, pad tokens zero, so a
// GEMM lane reads the scales of 4 consecutive tokens with one 16-byte load.
#include "vx_internal.h"

namespace vx {


// Mean and 1/sqrt(var + 1e-5) of one row, in the reference's summation order, broadcast to the wavefront.
__device__ inline void ln_stats(const float *__restrict__ xr, int d, int lane, float &mean, float &inv) {
    const int n8 = d / 8 * 8;
    float s = 0.0f;
    if (lane < 8)
        for (int c = lane; c < n8; c += 8) s += xr[c];  // lane l < 4: s0[l]; lane 4 + l: s1[l]
    float p = s + __shfl(s, lane + 4, 64);              // lanes 0-3: s0[l] + s1[l]
    float sum = (p + __shfl(p, 1, 64)) + (__shfl(p, 2, 64) + __shfl(p, 3, 64));
    for (int c = n8; c < d; c++) sum += xr[c];
    sum = __shfl(sum, 0, 64);
    mean = sum / (float)d;
    float q = 0.0f;
    if (lane < 8)
        for (int c = lane; c < n8; c += 8) {
            const float a = xr[c] - mean;
            q = __builtin_fmaf(a, a, q);
        }
    p = q + __shfl(q, lane + 4, 64);
    float sq = (p + __shfl(p, 1, 64)) + (__shfl(p, 2, 64) + __shfl(p, 3, 64));
    for (int c = n8; c < d; c++) {
        const float a = xr[c] - mean;
        sq += a * a;
    }
    sq = __shfl(sq, 0, 64);
    const float var = sq / (float)d;
    inv = 1.0f / __builtin_sqrtf(var + 1e-5f);
}

// y = ((x - mean) * inv) * g + b, one IEEE step at a time
__device__ inline float ln_apply(float x, float mean, float inv, float g, float b) { return (x - mean) * inv * g + b; }

// Fast path: group = 16 * L with L a power of two up to 64 lanes, or a multiple of 1024. Each lane owns 16
// consecutive values of a 1024-wide chunk; a group is L adjacent lanes (or whole chunks), reduced with xor
// shuffles inside the lane group.
template <int L, bool LN>
__global__ __launch_bounds__(256) void quantize_fast_kernel(const float *__restrict__ x, int n, int inp, int group,
                                                          int np, int8_t *__restrict__ q, float *__restrict__ st,
                                                          int32_t *__restrict__ gt, const float *__restrict__ lg,
                                                          const float *__restrict__ lb) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;  // uniform per wavefront
    const float *xr = x + (int64_t)t * inp;
    float mean = 0.0f, linv = 1.0f;
    if constexpr (LN) ln_stats(xr, inp, lane, mean, linv);
    // the 16 values of one lane at column `base`, normalized when LN
    auto load16 = [&](int base, float (&v)[16]) {
        const float4 *p = (const float4 *)(xr + base);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = p[i];
            v[4 * i] = f.x;
            v[4 * i + 1] = f.y;
            v[4 * i + 2] = f.z;
            v[4 * i + 3] = f.w;
        }
        if constexpr (LN) {
            const float4 *pg = (const float4 *)(lg + base), *pb = (const float4 *)(lb + base);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 g4 = pg[i], b4 = pb[i];
                v[4 * i] = ln_apply(v[4 * i], mean, linv, g4.x, b4.x);
                v[4 * i + 1] = ln_apply(v[4 * i + 1], mean, linv, g4.y, b4.y);
                v[4 * i + 2] = ln_apply(v[4 * i + 2], mean, linv, g4.z, b4.z);
                v[4 * i + 3] = ln_apply(v[4 * i + 3], mean, linv, g4.w, b4.w);
            }
        }
    };
    int8_t *qr = q + (int64_t)t * inp;
    const int ng = inp / group;
    const int chunks_per_group = group >= 1024 ? group / 1024 : 1;
    for (int c0 = 0; c0 < inp; c0 += 1024 * chunks_per_group) {
        // amax over this lane's values of the group (all chunks of the group)
        float m = 0.0f;
        for (int cc = 0; cc < chunks_per_group; cc++) {
            const int base = c0 + cc * 1024 + lane * 16;
            if (base < inp) {
                float v[16];
                load16(base, v);
#pragma unroll
                for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[i]));
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
                float v[16];
                load16(base, v);
                uint32_t w[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int8_t c0_ = code_of(v[4 * i], inv), c1 = code_of(v[4 * i + 1], inv),
                                 c2 = code_of(v[4 * i + 2], inv), c3 = code_of(v[4 * i + 3], inv);
                    sum += (int)c0_ + (int)c1 + (int)c2 + (int)c3;
                    w[i] = (uint32_t)(uint8_t)c0_ | ((uint32_t)(uint8_t)c1 << 8) | ((uint32_t)(uint8_t)c2 << 16) |
                           ((uint32_t)(uint8_t)c3 << 24);
                }
                store16_sep((uint4 *)(qr + base), make_uint4(w[0], w[1], w[2], w[3]));
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

// Row-resident path: inp = NC * 1024 (NC <= 4), one wavefront per token, the row loaded once into registers
// (16 consecutive floats per lane per 1024-column chunk). With LN the row is also staged in the wavefront's LDS
// slot, where lanes 0-7 run the reference-order statistics. MODE 0 quantizes, MODE 1 writes the LayerNorm row as
// float32 (y), MODE 2 writes that row to y and then quantizes its LayerNorm with (lg2, lb2): a layer's norm_out
// followed by the next layer's first LayerNorm->quantize in one pass. Waves of pad tokens [n, np) only write zero
// scales and code sums, so no pad launch is needed. KEEP (one 1024-column row): the row's LDS column is held in 128
// registers between the two statistics chains (the shortest chain latency, two wavefronts per SIMD); without it
// the chains read it in quarters and the kernel fits four wavefronts per SIMD, for launches with many rows.
template <int L, int NC, bool LN, int MODE, bool KEEP = true>
__global__ __launch_bounds__(256, KEEP ? 1 : 4) void quant_rows_kernel(const float *__restrict__ x, int n, int np, int group,
                                                        int8_t *__restrict__ q, float *__restrict__ st,
                                                        int32_t *__restrict__ gt, const float *__restrict__ lg,
                                                        const float *__restrict__ lb, float *__restrict__ y,
                                                        const float *__restrict__ lg2,
                                                        const float *__restrict__ lb2) {
    static_assert(MODE != 2 || LN, "MODE 2 is two LayerNorms");
    constexpr int inp = NC * 1024;
    // the transposed row of each wavefront: 8 residue rows of inp / 8 values, each padded by 4 floats so that the
    // 16-byte reads of lanes 0-7 fall on distinct LDS banks
    constexpr int KLP = inp / 8 + 4;
    __shared__ __attribute__((aligned(16))) float srow[LN ? 4 : 1][LN ? 8 * KLP : 4];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + w;
    if (t >= np) return;
    const int ng = inp / group;
    if (t >= n) {
        if (MODE != 1)
            for (int g = lane; g < ng; g += 64) {
                st[(int64_t)g * np + t] = 0.0f;
                gt[(int64_t)g * np + t] = 0;
            }
        return;
    }
    const float *xr = x + (int64_t)t * inp;
    float4 lgv[LN ? NC : 1][4], lbv[LN ? NC : 1][4];  // gamma / beta quads, fetched with the row
    float4 lgv2[MODE == 2 ? NC : 1][4], lbv2[MODE == 2 ? NC : 1][4];
    if constexpr (LN) {
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lgv[c][i] = ((const float4 *)(lg + c * 1024 + lane * 16))[i];
                lbv[c][i] = ((const float4 *)(lb + c * 1024 + lane * 16))[i];
                if constexpr (MODE == 2) {
                    lgv2[c][i] = ((const float4 *)(lg2 + c * 1024 + lane * 16))[i];
                    lbv2[c][i] = ((const float4 *)(lb2 + c * 1024 + lane * 16))[i];
                }
            }
    }
    float v[NC][16];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        const float4 *p = (const float4 *)(xr + c * 1024 + lane * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = p[i];
            v[c][4 * i] = f.x;
            v[c][4 * i + 1] = f.y;
            v[c][4 * i + 2] = f.z;
            v[c][4 * i + 3] = f.w;
        }
    }
    // LayerNorm of the row in v, in place: statistics in the reference's order over the row staged in LDS
    auto ln_pass = [&](const float4 (&G)[LN ? NC : 1][4], const float4 (&B)[LN ? NC : 1][4]) __attribute__((always_inline)) {
        // the row transposed by column residue: T[j * KLP + k] = x[8k + j], so that the running sum of residue j
        // (the reference's lane j of row_mean_var_portable) walks contiguous memory
        constexpr int KL = inp / 8;
        float *T = srow[w];
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++)
                *(float2 *)(T + j * KLP + c * 128 + 2 * lane) = make_float2(v[c][j], v[c][8 + j]);
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's row is in LDS
        __builtin_amdgcn_wave_barrier();
        float mean, linv;
        // lane j < 8 keeps the running sum of columns j, j+8, j+16, ... in that order. Each 128-value stretch of
        // its column is read from LDS in one batch before the dependent additions start.
        float s = 0.0f;
        if constexpr (KL == 128 && KEEP) {
            // one stretch (1024 columns): all 32 reads issue before the first addition, and the stretch stays in
            // registers for the variance chain
            float4 f[32];
            if (lane < 8) {
                const float *r = T + lane * KLP;
#pragma unroll
                for (int k = 0; k < 32; k++) f[k] = *(const float4 *)(r + 4 * k);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int k = 0; k < 32; k++) {
                    s += f[k].x;
                    s += f[k].y;
                    s += f[k].z;
                    s += f[k].w;
                }
            }
            mean = hsum8_lanes(s) / (float)inp;
            float qs = 0.0f;
            if (lane < 8) {
#pragma unroll
                for (int k = 0; k < 32; k++) {
                    float a = f[k].x - mean;
                    qs = __builtin_fmaf(a, a, qs);
                    a = f[k].y - mean;
                    qs = __builtin_fmaf(a, a, qs);
                    a = f[k].z - mean;
                    qs = __builtin_fmaf(a, a, qs);
                    a = f[k].w - mean;
                    qs = __builtin_fmaf(a, a, qs);
                }
            }
            const float var = hsum8_lanes(qs) / (float)inp;
            linv = 1.0f / __builtin_sqrtf(var + 1e-5f);
        } else if constexpr (KL == 128) {
            // the same chains with the column read in quarters of 32 values (8 reads each)
            if (lane < 8) {
                const float *r = T + lane * KLP;
#pragma unroll
                for (int k0 = 0; k0 < 32; k0 += 8) {
                    float4 f[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) f[k] = *(const float4 *)(r + 4 * (k0 + k));
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        s += f[k].x;
                        s += f[k].y;
                        s += f[k].z;
                        s += f[k].w;
                    }
                }
            }
            mean = hsum8_lanes(s) / (float)inp;
            float qs = 0.0f;
            if (lane < 8) {
                const float *r = T + lane * KLP;
#pragma unroll
                for (int k0 = 0; k0 < 32; k0 += 8) {
                    float4 f[8];
#pragma unroll
                    for (int k = 0; k < 8; k++) f[k] = *(const float4 *)(r + 4 * (k0 + k));
#pragma unroll
                    for (int k = 0; k < 8; k++) {
                        float a = f[k].x - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].y - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].z - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].w - mean;
                        qs = __builtin_fmaf(a, a, qs);
                    }
                }
            }
            const float var = hsum8_lanes(qs) / (float)inp;
            linv = 1.0f / __builtin_sqrtf(var + 1e-5f);
        } else {
            if (lane < 8) {
                const float *r = T + lane * KLP;
#pragma unroll
                for (int k0 = 0; k0 < KL; k0 += 128) {
                    float4 f[32];
#pragma unroll
                    for (int k = 0; k < 32; k++) f[k] = *(const float4 *)(r + k0 + 4 * k);
#pragma unroll
                    for (int k = 0; k < 32; k++) {
                        s += f[k].x;
                        s += f[k].y;
                        s += f[k].z;
                        s += f[k].w;
                    }
                }
            }
            mean = hsum8_lanes(s) / (float)inp;
            float qs = 0.0f;
            if (lane < 8) {
                const float *r = T + lane * KLP;
#pragma unroll
                for (int k0 = 0; k0 < KL; k0 += 128) {
                    float4 f[32];
#pragma unroll
                    for (int k = 0; k < 32; k++) f[k] = *(const float4 *)(r + k0 + 4 * k);
#pragma unroll
                    for (int k = 0; k < 32; k++) {
                        float a = f[k].x - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].y - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].z - mean;
                        qs = __builtin_fmaf(a, a, qs);
                        a = f[k].w - mean;
                        qs = __builtin_fmaf(a, a, qs);
                    }
                }
            }
            const float var = hsum8_lanes(qs) / (float)inp;
            linv = 1.0f / __builtin_sqrtf(var + 1e-5f);
        }
#pragma unroll
        for (int c = 0; c < NC; c++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 g4 = G[c][i], b4 = B[c][i];
                v[c][4 * i] = ln_apply(v[c][4 * i], mean, linv, g4.x, b4.x);
                v[c][4 * i + 1] = ln_apply(v[c][4 * i + 1], mean, linv, g4.y, b4.y);
                v[c][4 * i + 2] = ln_apply(v[c][4 * i + 2], mean, linv, g4.z, b4.z);
                v[c][4 * i + 3] = ln_apply(v[c][4 * i + 3], mean, linv, g4.w, b4.w);
            }
        }
    };
    if constexpr (LN) ln_pass(lgv, lbv);
    if constexpr (MODE != 0) {
        float *yr = y + (int64_t)t * inp;
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                store16_sep((float4 *)(yr + c * 1024 + lane * 16 + 4 * i),
                            make_float4(v[c][4 * i], v[c][4 * i + 1], v[c][4 * i + 2], v[c][4 * i + 3]));
        if constexpr (MODE == 1) return;
    }
    if constexpr (MODE == 2) ln_pass(lgv2, lbv2);
    // groups of L lanes (group = 16 L columns) or whole chunks (L = 64, group = 1024 * k)
    int8_t *qr = q + (int64_t)t * inp;
    constexpr int CPG = 1;  // chunks per group when L == 64 is handled below
    (void)CPG;
    if (L < 64 || group == 1024) {
#pragma unroll
        for (int c = 0; c < NC; c++) {
            float m = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[c][i]));
            m = lane_group_max<L>(m);
            const float sc = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / sc;
            int sum = 0;
            uint32_t wd[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int8_t c0 = code_of(v[c][4 * i], inv), c1 = code_of(v[c][4 * i + 1], inv),
                             c2 = code_of(v[c][4 * i + 2], inv), c3 = code_of(v[c][4 * i + 3], inv);
                sum += (int)c0 + (int)c1 + (int)c2 + (int)c3;
                wd[i] = (uint32_t)(uint8_t)c0 | ((uint32_t)(uint8_t)c1 << 8) | ((uint32_t)(uint8_t)c2 << 16) |
                        ((uint32_t)(uint8_t)c3 << 24);
            }
            store16_sep((uint4 *)(qr + c * 1024 + lane * 16), make_uint4(wd[0], wd[1], wd[2], wd[3]));
            sum = lane_group_sum<L>(sum);
            if ((lane & (L - 1)) == 0) {
                const int g = (c * 1024 + lane * 16) / group;
                st[(int64_t)g * np + t] = sc;
                gt[(int64_t)g * np + t] = sum;
            }
        }
    } else {
        // one group spans several chunks (group = 1024 * k): reduce over the chunks of each group
        const int cpg = group / 1024;
        for (int c0 = 0; c0 < NC; c0 += cpg) {
            float m = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; c++)
                if (c >= c0 && c < c0 + cpg)
#pragma unroll
                    for (int i = 0; i < 16; i++) m = fmaxf(m, fabsf(v[c][i]));
            m = lane_group_max<64>(fmaxf(m, 0.0f));
            const float sc = m == 0.0f ? 1.0f : m / 127.0f;
            const float inv = 1.0f / sc;
            int sum = 0;
#pragma unroll
            for (int c = 0; c < NC; c++) {
                if (c < c0 || c >= c0 + cpg) continue;
                uint32_t wd[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int8_t a0 = code_of(v[c][4 * i], inv), a1 = code_of(v[c][4 * i + 1], inv),
                                 a2 = code_of(v[c][4 * i + 2], inv), a3 = code_of(v[c][4 * i + 3], inv);
                    sum += (int)a0 + (int)a1 + (int)a2 + (int)a3;
                    wd[i] = (uint32_t)(uint8_t)a0 | ((uint32_t)(uint8_t)a1 << 8) | ((uint32_t)(uint8_t)a2 << 16) |
                            ((uint32_t)(uint8_t)a3 << 24);
                }
                store16_sep((uint4 *)(qr + c * 1024 + lane * 16), make_uint4(wd[0], wd[1], wd[2], wd[3]));
            }
            sum = lane_group_sum<64>(sum);
            if (lane == 0) {
                const int g = c0 / cpg;
                st[(int64_t)g * np + t] = sc;
                gt[(int64_t)g * np + t] = sum;
            }
        }
    }
}

// Any group that divides inp: one group at a time across the wavefront.
template <bool LN>
__global__ __launch_bounds__(256) void quantize_generic_kernel(const float *__restrict__ x, int n, int inp,
                                                             int group, int np, int8_t *__restrict__ q,
                                                             float *__restrict__ st, int32_t *__restrict__ gt,
                                                             const float *__restrict__ lg,
                                                             const float *__restrict__ lb) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const float *xr = x + (int64_t)t * inp;
    int8_t *qr = q + (int64_t)t * inp;
    const int ng = inp / group;
    float mean = 0.0f, linv = 1.0f;
    if constexpr (LN) ln_stats(xr, inp, lane, mean, linv);
    auto val = [&](int k) { return LN ? ln_apply(xr[k], mean, linv, lg[k], lb[k]) : xr[k]; };
    for (int g = 0; g < ng; g++) {
        const int g0 = g * group;
        float m = 0.0f;
        for (int c = lane; c < group; c += 64) m = fmaxf(m, fabsf(val(g0 + c)));
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float s = m == 0.0f ? 1.0f : m / 127.0f;
        const float inv = 1.0f / s;
        int sum = 0;
        for (int c = lane; c < group; c += 64) {
            const int8_t code = code_of(val(g0 + c), inv);
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

// Launches the quantizer; with g and b, the LN variant (both NULL: plain quantization).
void quantize_ln(const float *x, int64_t n, int64_t inp, int64_t group, const float *g, const float *b, int8_t *q,
                 float *scales_t, int32_t *gsum_t, hipStream_t stream) {
    require(n == 0 || (x && q && scales_t && gsum_t), "x, q, scales_t and gsum_t must not be NULL");
    require((g == nullptr) == (b == nullptr), "LayerNorm needs both gamma and beta");
    require(n >= 0 && inp > 0 && group > 0 && inp % group == 0, "inp must be a positive multiple of group");
    require(n * inp < (1ll << 31), "activation block above 2 GiB");
    if (n == 0) return;
    const bool ln = g != nullptr;
    const int np = (int)((n + 15) / 16 * 16), ng = (int)(inp / group);
    const unsigned blocks = (unsigned)((n + 3) / 4);
    const int ni = (int)n, ii = (int)inp, gi = (int)group;
    auto al16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool aligned = al16(x) && al16(q) && inp % 1024 == 0 && (!ln || (al16(g) && al16(b)));
    int L = 0;
    if (aligned) {
        if (group % 1024 == 0)
            L = 64;
        else if (group >= 64 && group <= 1024 && (group & (group - 1)) == 0)
            L = group / 16;
    }
    const int nc = (int)(inp / 1024);
    if (L != 0 && inp <= 4096) {  // the row-resident kernel covers the pad tokens too
        const unsigned blk = (unsigned)((np + 3) / 4);
#define VX_QR(LL, NC)                                                                                                \
    (ln ? quant_rows_kernel<LL, NC, true, 0> : quant_rows_kernel<LL, NC, false, 0>)<<<blk, 256, 0, stream>>>(       \
        x, ni, np, gi, q, scales_t, gsum_t, g, b, nullptr, nullptr, nullptr)
        // the model's LayerNorm (1024 columns, 128-column groups) over many rows: four wavefronts per SIMD
        if (ln && L == 8 && nc == 1 && n > 1024) {
            quant_rows_kernel<8, 1, true, 0, false><<<blk, 256, 0, stream>>>(x, ni, np, gi, q, scales_t, gsum_t, g, b,
                                                                              nullptr, nullptr, nullptr);
            hip_check(hipGetLastError(), "quant_rows kernel launch");
            return;
        }
#define VX_QR_NC(LL)                                                                                                 \
    switch (nc) {                                                                                                    \
        case 1: VX_QR(LL, 1); break;                                                                                 \
        case 2: VX_QR(LL, 2); break;                                                                                 \
        case 3: VX_QR(LL, 3); break;                                                                                 \
        default: VX_QR(LL, 4); break;                                                                                \
    }
        switch (L) {
            case 4: VX_QR_NC(4); break;
            case 8: VX_QR_NC(8); break;
            case 16: VX_QR_NC(16); break;
            case 32: VX_QR_NC(32); break;
            default: VX_QR_NC(64); break;
        }
#undef VX_QR_NC
#undef VX_QR
        hip_check(hipGetLastError(), "quantize kernel launch");
        return;
    }
#define VX_QF(LL)                                                                                                    \
    (ln ? quantize_fast_kernel<LL, true> : quantize_fast_kernel<LL, false>)<<<blocks, 256, 0, stream>>>(           \
        x, ni, ii, gi, np, q, scales_t, gsum_t, g, b)
    switch (L) {
        case 4: VX_QF(4); break;
        case 8: VX_QF(8); break;
        case 16: VX_QF(16); break;
        case 32: VX_QF(32); break;
        case 64: VX_QF(64); break;
        default:
            (ln ? quantize_generic_kernel<true> : quantize_generic_kernel<false>)<<<blocks, 256, 0, stream>>>(
                x, ni, ii, gi, np, q, scales_t, gsum_t, g, b);
            break;
    }
#undef VX_QF
    hip_check(hipGetLastError(), "quantize kernel launch");
    if (np > n) {
        const int cnt = ng * (np - ni);
        quantize_pad_kernel<<<(cnt + 255) / 256, 256, 0, stream>>>(ni, np, ng, scales_t, gsum_t);
        hip_check(hipGetLastError(), "quantize pad kernel launch");
    }
}

void quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
              hipStream_t stream) {
    quantize_ln(x, n, inp, group, nullptr, nullptr, q, scales_t, gsum_t, stream);
}

// LayerNorm rows to f32 (tensor.rs:700-719), one wavefront per row.
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *__restrict__ x, int n, int d,
                                                        const float *__restrict__ g, const float *__restrict__ b,
                                                        float *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n) return;
    const float *xr = x + (int64_t)t * d;
    float mean, inv;
    ln_stats(xr, d, lane, mean, inv);
    float *yr = y + (int64_t)t * d;
    for (int k = lane; k < d; k += 64) yr[k] = ln_apply(xr[k], mean, inv, g[k], b[k]);
}

void layer_norm(const float *x, int64_t n, int64_t d, const float *g, const float *b, float *y, hipStream_t stream) {
    require(n == 0 || (x && g && b && y), "x, gamma, beta and y must not be NULL");
    require(n >= 0 && d > 0 && n * d < (1ll << 31), "bad LayerNorm shape");
    if (n == 0) return;
    auto al16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (d % 1024 == 0 && d <= 4096 && al16(x) && al16(y) && al16(g) && al16(b)) {
        const unsigned blk = (unsigned)((n + 3) / 4);
        const int ni = (int)n;
        switch (d / 1024) {
            case 1: quant_rows_kernel<4, 1, true, 1><<<blk, 256, 0, stream>>>(x, ni, ni, 64, nullptr, nullptr, nullptr, g, b, y, nullptr, nullptr); break;
            case 2: quant_rows_kernel<4, 2, true, 1><<<blk, 256, 0, stream>>>(x, ni, ni, 64, nullptr, nullptr, nullptr, g, b, y, nullptr, nullptr); break;
            case 3: quant_rows_kernel<4, 3, true, 1><<<blk, 256, 0, stream>>>(x, ni, ni, 64, nullptr, nullptr, nullptr, g, b, y, nullptr, nullptr); break;
            default: quant_rows_kernel<4, 4, true, 1><<<blk, 256, 0, stream>>>(x, ni, ni, 64, nullptr, nullptr, nullptr, g, b, y, nullptr, nullptr); break;
        }
        hip_check(hipGetLastError(), "layer_norm kernel launch");
        return;
    }
    layer_norm_kernel<<<(unsigned)((n + 3) / 4), 256, 0, stream>>>(x, (int)n, (int)d, g, b, y);
    hip_check(hipGetLastError(), "layer_norm kernel launch");
}

// A layer's norm_out (tensor.rs:700-719, encoder.rs:755) into y, then the next layer's first prepare_normed
// (norm_feed_forward1 -> quantize, ternary_linear.rs:132-155) of y, in one pass over each row: bit for bit as
// layer_norm followed by quantize_ln, with one launch and one read of the row fewer.
void layer_norm_quantize_ln(const float *x, int64_t n, int64_t d, const float *g, const float *b, float *y,
                            int64_t group, const float *g2, const float *b2, int8_t *q, float *scales_t,
                            int32_t *gsum_t, hipStream_t stream) {
    require(n == 0 || (x && g && b && y && g2 && b2 && q && scales_t && gsum_t), "LayerNorm -> quantize: NULL pointer");
    require(n >= 0 && d > 0 && group > 0 && d % group == 0 && n * d < (1ll << 31), "bad LayerNorm shape");
    if (n == 0) return;
    auto al16 = [](const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    const bool pow2 = group >= 64 && group <= 1024 && (group & (group - 1)) == 0;
    if (d % 1024 == 0 && d <= 4096 && pow2 && al16(x) && al16(y) && al16(g) && al16(b) && al16(g2) && al16(b2) &&
        al16(q)) {
        const int ni = (int)n, np = (int)((n + 15) / 16 * 16), gi = (int)group;
        const unsigned blk = (unsigned)((np + 3) / 4);
#define VX_LQ(LL, NC)                                                                                                \
    quant_rows_kernel<LL, NC, true, 2><<<blk, 256, 0, stream>>>(x, ni, np, gi, q, scales_t, gsum_t, g, b, y, g2, b2)
        if (group == 128 && d == 1024 && n > 1024) {  // many rows of the model's shape: four wavefronts per SIMD
            quant_rows_kernel<8, 1, true, 2, false><<<blk, 256, 0, stream>>>(x, ni, np, gi, q, scales_t, gsum_t, g, b,
                                                                              y, g2, b2);
            hip_check(hipGetLastError(), "LayerNorm -> quantize kernel launch");
            return;
        }
#define VX_LQ_NC(LL)                                                                                                 \
    switch (d / 1024) {                                                                                              \
        case 1: VX_LQ(LL, 1); break;                                                                                 \
        case 2: VX_LQ(LL, 2); break;                                                                                 \
        case 3: VX_LQ(LL, 3); break;                                                                                 \
        default: VX_LQ(LL, 4); break;                                                                                \
    }
        switch (group) {
            case 64: VX_LQ_NC(4); break;
            case 128: VX_LQ_NC(8); break;
            case 256: VX_LQ_NC(16); break;
            case 512: VX_LQ_NC(32); break;
            default: VX_LQ_NC(64); break;
        }
#undef VX_LQ_NC
#undef VX_LQ
        hip_check(hipGetLastError(), "LayerNorm -> quantize kernel launch");
        return;
    }
    layer_norm(x, n, d, g, b, y, stream);
    quantize_ln(y, n, d, group, g2, b2, q, scales_t, gsum_t, stream);
}

}  // namespace vx
