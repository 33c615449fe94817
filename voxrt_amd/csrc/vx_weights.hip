// vx_weights.hip — load-time upload and on-device repack of weight matrices (TernaryMatrix::from_packed_layout,
// packed.rs:73-130; from_i8_rows, packed.rs:164-201).
//
// The host hands over the thrush-ternary-v2 rows as stored in the model file (5 trits per byte, base 3, least
// significant digit first); one copy goes to the device and a kernel rewrites them into the MFMA operand order:
// per 16-row x 64-column block, lane l = 16*j + n of a wave owns one dword holding the 16 codes (trit + 1) of row
// n at columns 16*j .. 16*j+15, code of column 4*d + b at bit 8*b + 2*d. The GEMM then loads one coalesced dword
// per lane per MFMA and widens it with four shift/and operations.
#include <hip/hip_fp16.h>

#include <vector>

#include "vx_internal.h"

namespace vx {

__device__ inline int trit_code(const uint8_t *row, int64_t k) {
    // digit k % 5 of byte k / 5; the digit is the code (trit + 1)
    unsigned v = row[k / 5];
    switch (k % 5) {
        case 4: v /= 81; break;
        case 3: v /= 27; break;
        case 2: v /= 9; break;
        case 1: v /= 3; break;
        default: break;
    }
    return (int)(v % 3);
}

// One thread per output dword: (nb, kb, lane).
__global__ void repack_ternary_kernel(const uint8_t *__restrict__ q, int64_t out, int64_t inp, int64_t out_pad,
                                      uint32_t *__restrict__ codes) {
    int64_t nk = inp / 64;
    int64_t total = (out_pad / 16) * nk * 64;
    int64_t rb = (inp + 4) / 5;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int lane = (int)(i % 64);
        int64_t kb = (i / 64) % nk;
        int64_t nb = i / (64 * nk);
        int64_t row = nb * 16 + (lane % 16);
        int j = lane / 16;
        uint32_t v = 0;
        if (row < out) {
            const uint8_t *r = q + row * rb;
            for (int d = 0; d < 4; d++)
                for (int b = 0; b < 4; b++) {
                    int64_t k = kb * 64 + 16 * j + 4 * d + b;
                    v |= (uint32_t)trit_code(r, k) << (8 * b + 2 * d);
                }
        } else {
            v = 0x55555555u;  // code 1 = trit 0 in every field
        }
        codes[i] = v;
    }
}

// One thread per output 16-byte chunk: (nb, kb, lane).
__global__ void repack_i8_kernel(const int8_t *__restrict__ rows, int64_t out, int64_t inp, int64_t out_pad,
                                 v4i *__restrict__ dst) {
    int64_t nk = inp / 64;
    int64_t total = (out_pad / 16) * nk * 64;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int lane = (int)(i % 64);
        int64_t kb = (i / 64) % nk;
        int64_t nb = i / (64 * nk);
        int64_t row = nb * 16 + (lane % 16);
        v4i v = {0, 0, 0, 0};
        if (row < out) v = *(const v4i *)(rows + row * inp + kb * 64 + 16 * (lane / 16));
        dst[i] = v;
    }
}

// scales_t[g][o] = scale of row o, group g (0 for pad rows); f16 -> f32 is exact.
__global__ void scales_f16_kernel(const __half *__restrict__ s, int64_t out, int64_t ng, int64_t out_pad,
                                  float *__restrict__ st) {
    int64_t total = ng * out_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t g = i / out_pad, o = i % out_pad;
        st[i] = o < out ? __half2float(s[o * ng + g]) : 0.0f;
    }
}

__global__ void scales_f32_kernel(const float *__restrict__ s, int64_t out, int64_t ng, int64_t out_pad,
                                  float *__restrict__ st) {
    int64_t total = ng * out_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        int64_t g = i / out_pad, o = i % out_pad;
        st[i] = o < out ? s[o * ng + g] : 0.0f;
    }
}

namespace {

struct DevBuf {
    void *p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

void *dev_alloc(size_t bytes) {
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        throw Error(VX_ERR_OOM, std::string("hipMalloc(") + std::to_string(bytes) + "): " + hipGetErrorString(e));
    }
    return p;
}

void check_shape(int64_t out, int64_t inp, int64_t group) {
    require(out > 0 && inp > 0 && group > 0, "out, inp and group must be positive");
    require(inp % group == 0, "inp must be a multiple of group");
    require(group % 64 == 0, "group must be a multiple of 64 (one i8 MFMA step)");
}

vx_tmat *new_tmat(int64_t out, int64_t inp, int64_t group, bool ternary) {
    vx_tmat *h = new vx_tmat;
    TMat *m = &h->m;
    m->out = out;
    m->inp = inp;
    m->group = group;
    m->ng = inp / group;
    m->out_pad = (out + kRowPad - 1) / kRowPad * kRowPad + kRowPad;
    m->ternary = ternary;
    return h;
}

int grid_for(int64_t total) {
    int64_t b = (total + 255) / 256;
    return (int)(b < 16384 ? (b > 0 ? b : 1) : 16384);
}

}  // namespace

vx_tmat *upload_packed(const uint8_t *qweight, const void *scales, bool scales_f16, int64_t out, int64_t inp,
                       int64_t group) {
    check_shape(out, inp, group);
    require(qweight && scales, "qweight and scales must not be NULL");
    vx_tmat *h = new_tmat(out, inp, group, true);
    TMat *m = &h->m;
    try {
        int64_t rb = (inp + 4) / 5;
        DevBuf q, s;
        q.p = dev_alloc((size_t)(out * rb));
        size_t sbytes = (size_t)(out * m->ng) * (scales_f16 ? 2 : 4);
        s.p = dev_alloc(sbytes);
        hip_check(hipMemcpy(q.p, qweight, (size_t)(out * rb), hipMemcpyHostToDevice), "hipMemcpy(qweight)");
        hip_check(hipMemcpy(s.p, scales, sbytes, hipMemcpyHostToDevice), "hipMemcpy(scales)");
        int64_t ncodes = (m->out_pad / 16) * (inp / 64) * 64;
        m->wdev = dev_alloc((size_t)ncodes * 4);
        m->scales_t = (float *)dev_alloc((size_t)(m->ng * m->out_pad) * 4);
        repack_ternary_kernel<<<grid_for(ncodes), 256>>>((const uint8_t *)q.p, out, inp, m->out_pad,
                                                         (uint32_t *)m->wdev);
        hip_check(hipGetLastError(), "repack_ternary_kernel launch");
        if (scales_f16)
            scales_f16_kernel<<<grid_for(m->ng * m->out_pad), 256>>>((const __half *)s.p, out, m->ng, m->out_pad,
                                                                      m->scales_t);
        else
            scales_f32_kernel<<<grid_for(m->ng * m->out_pad), 256>>>((const float *)s.p, out, m->ng, m->out_pad,
                                                                      m->scales_t);
        hip_check(hipGetLastError(), "scales kernel launch");
        hip_check(hipDeviceSynchronize(), "weight repack");
    } catch (...) {
        if (m->wdev) (void)hipFree(m->wdev);
        if (m->scales_t) (void)hipFree(m->scales_t);
        delete h;
        throw;
    }
    return h;
}

// A TernaryMatrix already unpacked to trits (int8 rows in {-1, 0, +1}, packed.rs:48-60 in the Rows layout) with f32
// scales: packed back into the model file's base-3 rows on the host (5 trits per byte, least significant digit
// first, digit = trit + 1, pad digits 0: trits.rs:30-41) and uploaded through the same device repack, so the device
// matrix is the ternary 2-bit one. A value outside {-1, 0, +1} is refused.
vx_tmat *upload_trits(const int8_t *trits, const float *scales, int64_t out, int64_t inp, int64_t group) {
    check_shape(out, inp, group);
    require(trits && scales, "trits and scales must not be NULL");
    const int64_t rb = (inp + 4) / 5;
    std::vector<uint8_t> packed((size_t)(out * rb), 0);
    for (int64_t o = 0; o < out; o++) {
        const int8_t *row = trits + o * inp;
        uint8_t *dst = packed.data() + o * rb;
        for (int64_t b = 0; b < rb; b++) {
            int v = 0;
            for (int d = 4; d >= 0; d--) {
                const int64_t c = b * 5 + d;
                int digit = 0;
                if (c < inp) {
                    const int t = row[c];
                    require(t >= -1 && t <= 1, "trits must be -1, 0 or +1 (row " + std::to_string(o) + ")");
                    digit = t + 1;
                }
                v = v * 3 + digit;
            }
            dst[b] = (uint8_t)v;
        }
    }
    return upload_packed(packed.data(), scales, false, out, inp, group);
}

vx_tmat *upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group) {
    check_shape(out, inp, group);
    require(rows && scales, "rows and scales must not be NULL");
    vx_tmat *h = new_tmat(out, inp, group, false);
    TMat *m = &h->m;
    try {
        DevBuf r, s;
        r.p = dev_alloc((size_t)(out * inp));
        s.p = dev_alloc((size_t)(out * m->ng) * 4);
        hip_check(hipMemcpy(r.p, rows, (size_t)(out * inp), hipMemcpyHostToDevice), "hipMemcpy(rows)");
        hip_check(hipMemcpy(s.p, scales, (size_t)(out * m->ng) * 4, hipMemcpyHostToDevice), "hipMemcpy(scales)");
        int64_t nchunks = (m->out_pad / 16) * (inp / 64) * 64;
        m->wdev = dev_alloc((size_t)nchunks * 16);
        m->scales_t = (float *)dev_alloc((size_t)(m->ng * m->out_pad) * 4);
        repack_i8_kernel<<<grid_for(nchunks), 256>>>((const int8_t *)r.p, out, inp, m->out_pad, (v4i *)m->wdev);
        hip_check(hipGetLastError(), "repack_i8_kernel launch");
        scales_f32_kernel<<<grid_for(m->ng * m->out_pad), 256>>>((const float *)s.p, out, m->ng, m->out_pad,
                                                                  m->scales_t);
        hip_check(hipGetLastError(), "scales kernel launch");
        hip_check(hipDeviceSynchronize(), "weight repack");
    } catch (...) {
        if (m->wdev) (void)hipFree(m->wdev);
        if (m->scales_t) (void)hipFree(m->scales_t);
        delete h;
        throw;
    }
    return h;
}

void free_tmat(vx_tmat *h) {
    if (!h) return;
    if (h->m.wdev) (void)hipFree(h->m.wdev);
    if (h->m.scales_t) (void)hipFree(h->m.scales_t);
    delete h;
}

}  // namespace vx
