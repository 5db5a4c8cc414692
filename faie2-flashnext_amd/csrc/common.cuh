// Shared device helpers and host error plumbing for libfaie2fn (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace fn {

// ---------------------------------------------------------------------------------------------
// host errors: the reference convention (engine/faie2fn.cu:111-118): entry points return 0 or -1 and leave the
// message in one process-global string read through fn_error().

void set_error(const std::string &msg);
const char *error_cstr();

#define FN_CK(x)                                                                                           \
    do {                                                                                                   \
        hipError_t e_ = (x);                                                                               \
        if (e_ != hipSuccess) {                                                                            \
            ::fn::set_error(std::string(#x) + " -> " + hipGetErrorString(e_));                             \
            return -1;                                                                                     \
        }                                                                                                  \
    } while (0)
#define FN_FAIL(msg)                                                                                       \
    do {                                                                                                   \
        ::fn::set_error(msg);                                                                              \
        return -1;                                                                                         \
    } while (0)

// compute units of the current device (queried once; 256, MI355X, if the query fails)
int device_cus();

// ---------------------------------------------------------------------------------------------
// wave64 cross-lane primitives.  Rotations inside a row of 16 lanes go through DPP (row_ror), the exchange
// between the two rows of each 32-lane half through ds_swizzle (bit mode, xor 16), and the two halves of the
// wave are joined with v_readlane, so a full-wave reduction touches neither LDS memory nor a barrier.

template <int N> __device__ __forceinline__ float dpp_ror(float v) {
    static_assert(N >= 1 && N <= 15, "row_ror takes 1..15");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xf, 0xf,
                                                                 false));
}

// value of lane l ^ 16 (ds_swizzle bit mode: and_mask 0x1f, or_mask 0, xor_mask 0x10)
__device__ __forceinline__ float swz_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f));
}

// value of lane l ^ 32 (a lane permute through the LDS crossbar, no LDS memory)
__device__ __forceinline__ float shfl_xor32(float v) { return __shfl_xor(v, 32); }

// sum over the 16 lanes of each row, returned to every lane of the row (every lane gets the same bits)
__device__ __forceinline__ float row_sum(float v) {
    v += dpp_ror<8>(v);
    v += dpp_ror<4>(v);
    v += dpp_ror<2>(v);
    v += dpp_ror<1>(v);
    return v;
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_ror<8>(v));
    v = fmaxf(v, dpp_ror<4>(v));
    v = fmaxf(v, dpp_ror<2>(v));
    v = fmaxf(v, dpp_ror<1>(v));
    return v;
}
// sum over each 32-lane half, returned to every lane of the half
__device__ __forceinline__ float half_sum(float v) {
    v = row_sum(v);
    return v + swz_xor16(v);
}
__device__ __forceinline__ float readlane(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// sum / max over all 64 lanes, wave-uniform result (call from wave-uniform control flow)
__device__ __forceinline__ float wave_sum(float v) {
    v = half_sum(v);
    return readlane(v, 0) + readlane(v, 32);
}
__device__ __forceinline__ float wave_max(float v) {
    v = row_max(v);
    v = fmaxf(v, swz_xor16(v));
    return fmaxf(readlane(v, 0), readlane(v, 32));
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

__device__ __forceinline__ float4 f4(float a) { return make_float4(a, a, a, a); }

// 16-byte loads and stores with the nontemporal hint (data touched once per call: keep it out of the caches'
// reuse path)
typedef float v4f_ __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4 *p) {
    const v4f_ v = __builtin_nontemporal_load(reinterpret_cast<const v4f_ *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4 *p, float4 x) {
    v4f_ v = {x.x, x.y, x.z, x.w};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f_ *>(p));
}

}  // namespace fn
