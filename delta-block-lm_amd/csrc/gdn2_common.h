// Shared device-side helpers for the gfx950 GDN-2 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn2.h"

namespace gdn2 {

// Device copy of a gdn2_view: base pointer plus element strides.
struct View {
    const void *data;
    int64_t s0, s1, s2, s3;
};

inline View make_view(const gdn2_view *v) {
    View out{};
    if (v) {
        out.data = v->data;
        out.s0 = v->stride[0];
        out.s1 = v->stride[1];
        out.s2 = v->stride[2];
        out.s3 = v->stride[3];
    }
    return out;
}

typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t x) {
    return __uint_as_float(((uint32_t)x) << 16);
}

// Round to nearest even (gfx950 v_cvt_pk_bf16_f32; NaN stays NaN).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
}

template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float load(const void *p, int64_t i) {
        return reinterpret_cast<const float *>(p)[i];
    }
    static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
        reinterpret_cast<float *>(p)[i] = x;
    }
};
template <> struct Elem<bf16_t> {
    static __device__ __forceinline__ float load(const void *p, int64_t i) {
        return bf16_to_f32(reinterpret_cast<const bf16_t *>(p)[i]);
    }
    static __device__ __forceinline__ void store(void *p, int64_t i, float x) {
        reinterpret_cast<bf16_t *>(p)[i] = f32_to_bf16(x);
    }
};

template <typename T>
__device__ __forceinline__ float ld4(const View &v, int64_t a, int64_t b, int64_t c, int64_t d) {
    return Elem<T>::load(v.data, a * v.s0 + b * v.s1 + c * v.s2 + d * v.s3);
}

__device__ __forceinline__ void store_out(void *p, int bf16, int64_t i, float x) {
    if (bf16) Elem<bf16_t>::store(p, i, x);
    else Elem<float>::store(p, i, x);
}

}  // namespace gdn2
