// Internal API of the path engine (engine.hip); the C ABI wrappers live in api.hip.
#pragma once

#include "../../include/faie2fn.h"
#include "gdn.h"

namespace fn {

int path_init(int B, int nl, int attn_every, int nkh, int nvh, int nq, int nkv, int max_ctx, int head_map,
              int gate_act, int nsplit);
int path_buffer(int il, int kind, void **ptr, size_t *bytes);
int path_step(int steps, float *ms);
int path_reset();
int path_use_graphs(int on);
void path_free();
bool path_loaded();
int path_n_past();
double path_dev_gb();
double path_last_ms();

}  // namespace fn
