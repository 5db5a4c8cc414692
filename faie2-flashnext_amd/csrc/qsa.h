// Internal API of the QSA indexer (qsa.hip) and the sparse attention launch (attn.hip).
#pragma once

#include "gdn.h"

namespace fn {

struct QsaIndexer {
    int B, nt, max_ctx, top, nrot;
    float theta, eps;
    const int32_t *pos;
    const float *iqk;       // [B][nt][4 * 128 + 128]: indexer query heads, then the raw index key
    const float *wqn, *wkn; // [128]
    float *IKc;             // [B][max_ctx][128] raw index keys
    float *BKc;             // [B][max_ctx / 4 / 64][32][64][4] block keys
    unsigned *status = nullptr;  // where kernels record misuse (FN_STATUS_*); null: the device's status word
};

size_t qsa_work_bytes(int B, int nt, int max_ctx, int top);
// indexer prep + scores + selection; on return *keys / *nkeys point into work (visible-key list per query)
int qsa_select_launch(const QsaIndexer &p, float *work, size_t work_bytes, const int32_t **keys, const int32_t **nkeys,
                      hipStream_t st);
int qsa_blocks_launch(const QsaIndexer &p, int j0, int j1, hipStream_t st);

// sparse GQA decode: the attention of AttnDecode restricted to the keys the indexer selects
size_t attn_qsa_work_bytes(int B, int nq, int nt, int hd, int nsplit, int max_ctx, int top);
int attn_qsa_launch(const AttnDecode &p, const QsaIndexer &ix, hipStream_t st);

}  // namespace fn
