// Internal launch API of the DeltaNet and attention kernels (device pointers, caller stream).
#pragma once

#include "../../include/faie2fn.h"
#include "common.cuh"

#include <algorithm>

namespace fn {

struct GdnBlock {
    int B, nkh, nvh, dk, dv, head_map, gate_act, nt, ring;
    float eps;
    const int32_t *pos;                 // [B] tokens already seen (conv ring index)
    const float *qkv;                   // [B][nt][C]
    const float *conv_w;                // [C][4]
    float *conv_ring;                   // [B][ring][C]
    const float *ab;                    // [B][nt][2 nvh]
    const float *dt_bias, *ssm_a;       // [nvh]
    float *S;                           // [B][nvh][dk][dv]
    const float *z;                     // [B][nt][nvh dv]
    const float *norm_w;                // [dv]
    float *out;                         // [B][nt][nvh dv]
    // alpha/beta projection fused into the block (nt = 1; ab unused): ab = wab . x, x [B][hidden] fp32,
    // wab [2 nvh][hidden] BF16 rows (alpha rows then beta rows)
    const float *x = nullptr;
    const uint16_t *wab = nullptr;
    int hidden = 0;
};

struct GdnCore {
    int B, nkh, nvh, dk, dv, head_map, nt;
    const float *q, *k;                 // [B][nt][nkh][dk]
    const float *v;                     // [B][nt][nvh][dv]
    const float *beta, *g;              // [B][nt][nvh]
    float *S;                           // [B][nvh][dk][dv]
    float *o;                           // [B][nt][nvh][dv]
};

// A verify step with deferred commit: blk.pos[b] is the position of the first new token; the kr[b] <= rnt tokens
// before it (positions pos - kr .. pos - 1) are the previous call's, replayed from rqkv [B][rnt][C] and
// rab [B][rnt][2 nvh] into the committed state first; the blk.nt new tokens get outputs and leave state untouched.
struct GdnVerify {
    GdnBlock blk;
    const int32_t *kr;
    int rnt;
    const float *rqkv, *rab;
};

int gdn_block_launch(const GdnBlock &p, hipStream_t st);
int gdn_verify_launch(const GdnVerify &p, hipStream_t st);
int gdn_core_launch(const GdnCore &p, hipStream_t st);

struct AttnDecode {
    int B, nq, nkv, hd, nrot, nt, max_ctx, nsplit;
    float theta, eps;
    const int32_t *pos;                 // [B] tokens already in the cache
    const float *qg;                    // [B][nt][nq][2][hd] query then gate
    const float *k, *v;                 // [B][nt][nkv][hd] new rows
    const float *wq, *wk;               // [hd]
    float *Kc, *Vc;                     // device cache layouts (see attn.hip)
    float *work;                        // attn_work_bytes()
    size_t work_bytes;
    float *og;                          // [B][nt][nq][hd]
    unsigned *status = nullptr;         // where kernels record misuse (FN_STATUS_*); null: the device's status word
};

size_t attn_work_bytes(int B, int nq, int nt, int hd, int nsplit);
int attn_pick_nsplit(int B, int nkv, int nt, int ctx);
int attn_decode_launch(const AttnDecode &p, hipStream_t st);
int advance_launch(int32_t *pos, int B, int nt, hipStream_t st);
int advance_by_launch(int32_t *pos, const int32_t *kr, int B, hipStream_t st);  // pos[b] += kr[b]

// Per-device status word (FN_STATUS_* bits of include/faie2fn.h): its device address for kernel arguments, and a
// read (after a device synchronize) that optionally clears it.  Not for use under stream capture.
int status_word(unsigned **out);
int status_read(unsigned *bits, bool clear);

int fill_normal_launch(float *p, size_t n, uint64_t seed, float mean, float std, hipStream_t st);
int copy_launch(void *dst, const void *src, size_t bytes, hipStream_t st);
int stage_events(void **ev, int n);

}  // namespace fn
