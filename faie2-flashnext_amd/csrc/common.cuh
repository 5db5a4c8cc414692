// Shared device helpers and host error plumbing for libfaie2fn (gfx950 / CDNA4, wave64).
#pragma once

#include <climits>

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

// Per-kernel timing without a profiler: while a list of events is set (fn_stage_events), the attention paths
// record the next event of the list on the call's stream after each of their launches; stage_mark does nothing
// when no list is set or the list is used up.  Not for graph capture.
void stage_mark(hipStream_t st);

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

// minimum over the 64 lanes (DPP inside rows, a swizzle across the row pair, readlanes across the halves),
// wave-uniform; call from wave-uniform control flow
__device__ __forceinline__ int wave_min_i(int v) {
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x128, 0xf, 0xf, false));  // row_ror 8
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x124, 0xf, 0xf, false));  // row_ror 4
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x122, 0xf, 0xf, false));  // row_ror 2
    v = min(v, __builtin_amdgcn_update_dpp(0, v, 0x121, 0xf, 0xf, false));  // row_ror 1
    v = min(v, __builtin_amdgcn_ds_swizzle(v, 0x401f));                     // lane ^ 16
    return min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 32));
}

// inclusive prefix sum over the wave in lane order through DPP alone (no LDS crossbar): row_shr 1, 2, 4, 8 scan each
// row of 16 lanes (lanes without a source read 0), row_bcast 15 carries row 0's total into row 1 and row 2's into
// row 3, row_bcast 31 carries lane 31's into rows 2 and 3.  Call from wave-uniform control flow.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr 1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr 2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr 4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr 8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast 15 into rows 1 and 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast 31 into rows 2 and 3
    return x;
}

// (value, index) of the better of two: larger value, ties to the lower index
__device__ __forceinline__ void vi_max(float &v, int &i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) {
        v = v2;
        i = i2;
    }
}

// (value, index) maximum over the wave, ties to the lower index, wave-uniform: the largest value, then the least
// index among the lanes that hold it (two cross-lane reductions, no LDS traffic)
__device__ __forceinline__ void wave_argmax(float &v, int &i) {
    const float m = wave_max(v);
    i = wave_min_i(v == m ? i : INT_MAX);
    v = m;
}

// maximum of a 64-bit key over the wave, wave-uniform, through DPP alone (no LDS crossbar): row_shr 1, 2, 4, 8 leave
// each row's maximum in its lane 15, row_bcast 15 and row_bcast 31 join the rows, lane 63 holds the result.  Lanes
// without a DPP source read 0, the identity of an unsigned maximum.  Call from wave-uniform control flow.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    uint32_t hi = (uint32_t) (k >> 32), lo = (uint32_t) k;
#define FN_KEY_STEP(CTRL, ROWS)                                                                                \
    do {                                                                                                      \
        const uint32_t h2 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) hi, CTRL, ROWS, 0xf, true);       \
        const uint32_t l2 = (uint32_t) __builtin_amdgcn_update_dpp(0, (int) lo, CTRL, ROWS, 0xf, true);       \
        if ((((uint64_t) h2 << 32) | l2) > (((uint64_t) hi << 32) | lo)) {                                    \
            hi = h2;                                                                                          \
            lo = l2;                                                                                          \
        }                                                                                                     \
    } while (0)
    FN_KEY_STEP(0x111, 0xf);  // row_shr 1
    FN_KEY_STEP(0x112, 0xf);  // row_shr 2
    FN_KEY_STEP(0x114, 0xf);  // row_shr 4
    FN_KEY_STEP(0x118, 0xf);  // row_shr 8
    FN_KEY_STEP(0x142, 0xa);  // row_bcast 15: lane 15 of rows 0 and 2 into rows 1 and 3
    FN_KEY_STEP(0x143, 0xc);  // row_bcast 31: lane 31 into rows 2 and 3
#undef FN_KEY_STEP
    return ((uint64_t) (uint32_t) __builtin_amdgcn_readlane((int) hi, 63) << 32) |
           (uint32_t) __builtin_amdgcn_readlane((int) lo, 63);
}

// MoE routing of one token by one whole wave (faie2fn.cu:1747-1798): p = softmax of the NE <= 1024 router logits
// l[0..NE), picked in order probability descending with ties to the lower expert (repeated argmax), npick picks.
// Returns pick `want`'s expert to every lane; with sel / wsel non-null (npick = NEU) it also writes the NEU picks
// and their weights renormalized over them, sel[k] and wsel[k].  The probabilities ride in registers (expert
// lane + 64 j in slot j), one wave argmax per pick.
// PER: experts per lane, 8 (NE <= 512) or 16 (NE <= 1024).
constexpr int ROUTE_PER = 16;
template <int PER>
__device__ __forceinline__ int route_wave(const float *__restrict__ l, int NE, int npick, int want,
                                          int32_t *__restrict__ sel, float *__restrict__ wsel) {
    const int lane = threadIdx.x & 63;
    float v[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = lane + 64 * j;
        v[j] = e < NE ? l[e] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = lane + 64 * j < NE ? expf(v[j] - mx) : -1.0f;  // in [0, 1]; -1 none
    float mine = 0.0f;  // lane k keeps the k-th pick's probability
    int got = 0;
    for (int k = 0; k < npick; ++k) {
        float bv = v[0];
        int bi = lane;
#pragma unroll
        for (int j = 1; j < PER; ++j)
            if (v[j] > bv) {  // strict: the lane's lower expert wins a tie
                bv = v[j];
                bi = lane + 64 * j;
            }
        // one reduction of (value, index) as a 64-bit key: a probability's bits order like the probability (it is
        // >= 0), the complemented index puts the lower expert first on a tie, and 0 is no candidate
        {
            const uint64_t key = bv >= 0.0f ? ((uint64_t) __float_as_uint(bv) << 32) | (uint32_t) ~bi : 0;
            const uint64_t best = wave_max_key(key);
            bv = __uint_as_float((uint32_t) (best >> 32));
            bi = (int) ~(uint32_t) best;
        }
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (lane + 64 * j == bi) v[j] = -1.0f;  // taken
        if (lane == k) mine = bv;
        if (sel && lane == 0) sel[k] = bi;
        if (k == want) got = bi;
    }
    if (wsel) {
        float sum = 0.0f;
        for (int k = 0; k < npick; ++k) sum += readlane(mine, k);  // in pick order
        if (lane < npick) wsel[lane] = mine / sum;
    }
    return got;
}
__device__ __forceinline__ int route_pick(const float *__restrict__ l, int NE, int npick, int want,
                                          int32_t *__restrict__ sel, float *__restrict__ wsel) {
    return NE <= 512 ? route_wave<8>(l, NE, npick, want, sel, wsel) : route_wave<16>(l, NE, npick, want, sel, wsel);
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

// x.x^2 + x.y^2 + x.z^2 + x.w^2 as one fixed chain (a product, then three fmas), so that every kernel that sums
// squares of a stream gets the same bits whatever the compiler would contract
__device__ __forceinline__ float sumsq4(float4 v) {
    float q = v.x * v.x;
    q = __builtin_fmaf(v.y, v.y, q);
    q = __builtin_fmaf(v.z, v.z, q);
    return __builtin_fmaf(v.w, v.w, q);
}
// h + y s, one fma per component
__device__ __forceinline__ float4 add_scaled(float4 h, float4 y, float s) {
    return make_float4(__builtin_fmaf(y.x, s, h.x), __builtin_fmaf(y.y, s, h.y), __builtin_fmaf(y.z, s, h.z),
                       __builtin_fmaf(y.w, s, h.w));
}

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

// Raw buffer access: a descriptor over [p, p + bytes) in four SGPRs, addressed per access by a VGPR byte offset and
// an SGPR one.  A long-lived per-lane address is then one VGPR, where a pointer plus an index is a 64-bit VGPR pair
// that the compiler hoists out of a loop (and spills under pressure); and a wave-uniform address stays a vector load
// (counted in vmcnt), never a scalar one (lgkmcnt, which every LDS wait also drains).  Accesses past `bytes` read 0
// and drop writes (the hardware range check).  aux 2 sets the nontemporal bit.
typedef __amdgpu_buffer_rsrc_t brsrc;
__device__ __forceinline__ brsrc buf(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short) 0, (int) bytes, 0x00020000);
}
__device__ __forceinline__ float bld(brsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int) voff, (int) soff, 0));
}
// (whole-vector bit casts: this compiler's __builtin_bit_cast of a single ext_vector element reads element 0)
typedef unsigned v4u_ __attribute__((ext_vector_type(4)));
template <int AUX = 0> __device__ __forceinline__ float4 bld4(brsrc r, uint32_t voff, uint32_t soff) {
    const v4f_ v = __builtin_bit_cast(v4f_, __builtin_amdgcn_raw_buffer_load_b128(r, (int) voff, (int) soff, AUX));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void bst(brsrc r, uint32_t voff, uint32_t soff, float x) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), r, (int) voff, (int) soff, 0);
}
template <int AUX = 0> __device__ __forceinline__ void bst4(brsrc r, uint32_t voff, uint32_t soff, float4 x) {
    const v4f_ v = {x.x, x.y, x.z, x.w};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u_, v), r, (int) voff, (int) soff, AUX);
}

// Workgroup barrier that orders LDS only.  __syncthreads() also waits for every outstanding global load and store
// of the wave (s_waitcnt vmcnt(0)); this one waits for the wave's LDS and scalar-memory operations (lgkmcnt(0))
// only, so global loads issued ahead of it stay in flight across it.  For LDS exchanges: global memory written
// before it is not ordered for the other waves.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The values of lanes l & ~16 and l | 16 (swap16), or l & ~32 and l | 32 (swap32), through v_permlane16_swap /
// v_permlane32_swap (VALU lane swaps, no LDS round trip): swapping two copies of x leaves the pair in the same
// order in both lanes, so r.x + r.y or max(r.x, r.y) gives every lane of the pair the same bits, and r.x + r.y
// equals x + (x of lane l ^ 32) bit for bit.  Inline asm: this compiler's __builtin_amdgcn_permlane16_swap /
// 32_swap lowering folds an add or max of the two results into one result doubled.  The s_nop 1 covers the wait
// states a VALU write needs before a permlane reads it.  (Not volatile: a pure function of its input, free to move,
// so it does not order the surrounding code.)
__device__ __forceinline__ float2 swap16(float x) {
    float a = x, b = x;
    asm("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return make_float2(a, b);
}
__device__ __forceinline__ float2 swap32(float x) {
    float a = x, b = x;
    asm("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
    return make_float2(a, b);
}
// x + x of lane l ^ 32, the same bits in both lanes of the pair
__device__ __forceinline__ float add_xor32(float x) {
    const float2 r = swap32(x);
    return r.x + r.y;
}

}  // namespace fn
