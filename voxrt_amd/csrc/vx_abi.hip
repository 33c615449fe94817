// vx_abi.hip — the extern "C" entry points of libvoxrt_hip (declared in include/voxrt_hip.h).
//
// Every entry point catches what the C++ layer throws and turns it into a vx_status plus a thread-local message
// (the convention of crates/voxrt-ffi/src/lib.rs:61-74,97-107), so no exception crosses the ABI.
#include <cstring>
#include <string>

#include "vx_internal.h"

namespace vx {
vx_tmat *upload_packed(const uint8_t *qweight, const void *scales, bool scales_f16, int64_t out, int64_t inp,
                       int64_t group);
vx_tmat *upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group);
void free_tmat(vx_tmat *h);
void quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t, int32_t *gsum_t,
              hipStream_t stream);
void gemm(const TMat *w, const int8_t *xq, const float *xs_t, const int32_t *xg_t, int64_t n, float *y,
          const float *bias, int ep, float alpha, int32_t *gs, int64_t r0, int64_t r1, int64_t t0, int64_t t1,
          hipStream_t st);
}  // namespace vx

namespace {

thread_local std::string g_last_error;

template <class F>
vx_status guarded(F &&f) {
    try {
        f();
        g_last_error.clear();
        return VX_OK;
    } catch (const vx::Error &e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return VX_ERR_HIP;
    } catch (...) {
        g_last_error = "unknown error";
        return VX_ERR_HIP;
    }
}

bool is_gfx950(int device) {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) != hipSuccess) return false;
    return std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
}

const vx::TMat *unwrap(const vx_tmat *w) { return &w->m; }

}  // namespace

extern "C" {

const char *vx_last_error(void) { return g_last_error.c_str(); }

int vx_detect(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    for (int d = 0; d < n; d++)
        if (is_gfx950(d)) return 1;
    return 0;
}

vx_status vx_init(int device) {
    return guarded([&] {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
            (void)hipGetLastError();
            throw vx::Error(VX_ERR_NO_DEVICE, "no HIP device visible");
        }
        if (device < 0 || device >= n) throw vx::Error(VX_ERR_INVALID, "device index out of range");
        if (!is_gfx950(device)) throw vx::Error(VX_ERR_NO_DEVICE, "device is not gfx950 (MI355X)");
        vx::hip_check(hipSetDevice(device), "hipSetDevice");
    });
}

vx_status vx_tmat_upload_packed(const uint8_t *qweight, const uint16_t *scales_f16, int64_t out, int64_t inp,
                                int64_t group, vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_packed(qweight, scales_f16, true, out, inp, group);
    });
}

vx_status vx_tmat_upload_packed_f32(const uint8_t *qweight, const float *scales, int64_t out, int64_t inp,
                                    int64_t group, vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_packed(qweight, scales, false, out, inp, group);
    });
}

vx_status vx_tmat_upload_i8(const int8_t *rows, const float *scales, int64_t out, int64_t inp, int64_t group,
                            vx_tmat **w) {
    return guarded([&] {
        vx::require(w != nullptr, "output handle pointer must not be NULL");
        *w = nullptr;
        *w = vx::upload_i8(rows, scales, out, inp, group);
    });
}

void vx_tmat_free(vx_tmat *w) { vx::free_tmat(w); }

vx_status vx_tmat_info(const vx_tmat *w, int64_t *out, int64_t *inp, int64_t *group, int *ternary) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        const vx::TMat *m = unwrap(w);
        if (out) *out = m->out;
        if (inp) *inp = m->inp;
        if (group) *group = m->group;
        if (ternary) *ternary = m->ternary ? 1 : 0;
    });
}

vx_status vx_quantize(const float *x, int64_t n, int64_t inp, int64_t group, int8_t *q, float *scales_t,
                      int32_t *gsum_t, void *stream) {
    return guarded([&] { vx::quantize(x, n, inp, group, q, scales_t, gsum_t, (hipStream_t)stream); });
}

vx_status vx_gemm_ep(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t, int64_t n,
                     float *y, const float *bias, int ep, float alpha, int32_t *group_sums, void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        const vx::TMat *m = unwrap(w);
        vx::gemm(m, xq, xs_t, xgsum_t, n, y, bias, ep, alpha, group_sums, 0, m->out, 0, n, (hipStream_t)stream);
    });
}

vx_status vx_gemm_rows_range(const vx_tmat *w, const int8_t *xq, const float *xs_t, const int32_t *xgsum_t,
                             int64_t n, float *y, int64_t r0, int64_t r1, int64_t t0, int64_t t1, int ep, float alpha,
                             void *stream) {
    return guarded([&] {
        vx::require(w != nullptr, "weight matrix must not be NULL");
        vx::gemm(unwrap(w), xq, xs_t, xgsum_t, n, y, nullptr, ep, alpha, nullptr, r0, r1, t0, t1,
                 (hipStream_t)stream);
    });
}

}  // extern "C"
