// Internal API of the model engine (model.hip): fn_load / fn_forward and the engine entry points when a model is
// loaded.  The C ABI wrappers live in api.hip.
#pragma once

#include <cstdint>
#include <vector>

namespace fn {

// shapes read from the GGUF metadata (<arch>.* keys) and the token embedding
struct ModelDims {
    int D = 0, NL = 0, NH = 0, NKV = 0, HD = 0, NROT = 0, NE = 0, NEU = 0, FFE = 0, FFS = 0, DS = 0, NKH = 0, NVH = 0;
    int DINNER = 0, CONVCH = 0, conv = 0, attn_every = 0, HC = 0, HCR = 0, IXH = 0, IXD = 0, top = 0, VOCAB = 0;
    // per-layer n-gram embedding (PLE): the layers that have one, and its hashing and shapes
    std::vector<int> ple;
    int ple_layers = 0, ple_heads = 0, ple_hd = 0, ple_eos = -1;
    std::vector<int64_t> ple_mult, ple_off, ple_size;
    float theta = 0, eps = 0;
};

int model_load(const char *shard1, const char *shard2, int max_ctx);
int model_forward(const int32_t *tokens, int nt, float *logits, int32_t *argmax);
int model_debug_layers(float *out);
int model_reset();
int model_use_graphs(int on);
bool model_loaded();
void model_free();
int model_n_past();
double model_dev_gb();
double model_last_ms();
int model_layers();
int model_dims(ModelDims *d);
// parse a GGUF and read its model shapes without touching a device
int model_inspect(const char *path, ModelDims *d);

}  // namespace fn
