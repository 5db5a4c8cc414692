// Internal structures of the model engine (model.hip forward, model_load.hip loader, ngram.hip).
//
// Weights and state live in arenas: one device allocation for the model-wide tensors and one per layer, each carved
// into pieces at 256-byte offsets.  A piece is addressed by its slot (what the tensor does in this engine's forward);
// which slots a layer holds, the GGUF tensors they come from and their shapes are rows of one table
// (model_load.hip), so the loader is a walk over that table rather than a sequence of calls.
#pragma once

#include "gguf.h"
#include "model.h"
#include "quant.h"

#include <array>
#include <vector>

namespace fn {

constexpr int MAXT = 8;                     // tokens per forward (the reference's batch limit, faie2fn.cu:67)
constexpr int HDK = 256, DSK = 128;         // attention head dim, DeltaNet head dim (built sizes)
constexpr int IXH = 4, IXD = 128, IXR = 4;  // indexer heads, head dim, keys per block (built sizes)
constexpr int RING = 16;                    // DeltaNet conv ring slots (>= MAXT + 3, a power of two)
// n-gram embedding: the conv's taps reach 9 positions back (kernel 4, dilation 3); its input history and the token
// history are rings indexed by position modulo NG_RING, which must hold the reach plus one call's tokens
constexpr int NG_REACH = 9, NG_RING = 32, NG_MAXH = 64;
static_assert(NG_RING >= NG_REACH + MAXT && (NG_RING & (NG_RING - 1)) == 0, "n-gram ring");

// what a tensor is for
enum Slot : int {
    // model-wide: token table, LM head, the final hyper-connection read, the n-gram table
    TOK_EMBED, LM_HEAD, FIN_NORM, FIN_DOWN, FIN_UP, NG_TABLE,
    // each layer's two hyper-connection reads: before the mixer (R0) and before the FFN (R1); DOWN holds the
    // low-rank down rows with the stream-inject rows below them, read by one product
    R0_NORM, R0_DOWN, R0_UP, R1_NORM, R1_DOWN, R1_UP,
    // gated DeltaNet mixer: input projection (q | k | v), output-gate projection, decay and step-size projection
    // (alpha rows then beta rows), output projection, conv taps, dt bias, A, gated-norm weight; state and conv ring
    DN_IN, DN_ZPROJ, DN_AB, DN_OUT, DN_CONVW, DN_DT, DN_A, DN_NORMW, DN_STATE, DN_RING,
    // attention mixer: projections (q with its gate, k, v, o; the indexer's q rows with its k rows below), norms,
    // K / V caches (K key-tiled) and the indexer's raw and block keys
    AT_QG, AT_K, AT_V, AT_O, AT_IX, AT_QNORM, AT_KNORM, AT_IXQNORM, AT_IXKNORM, AT_KCACHE, AT_VCACHE, AT_IXKEYS,
    AT_IXBLOCKS,
    // FFN: router logits with the shared expert's gate logit as one more row, shared expert, routed experts
    FF_ROUTER, FF_SH_GATE, FF_SH_UP, FF_SH_DOWN, FF_X_GATE, FF_X_UP, FF_X_DOWN,
    // n-gram embedding layers: key and value projections, the gate's norms, the conv taps, the conv input ring
    NG_KEY, NG_VAL, NG_KNORM, NG_QNORM, NG_CNORM, NG_CONVW, NG_HIST,
    SLOT_COUNT
};

// a packed weight as the GEMV kernels take it
struct QW {
    QLayout L;
    const uint8_t *p = nullptr;
};

struct Piece {
    bool on = false;
    uint8_t form = 0;
    QLayout L;           // packed weights
    size_t off = 0;      // inside the arena
    size_t bytes = 0;
    size_t n = 0;        // floats (vectors and state)
    const GTensor *src[2] = {nullptr, nullptr};
    uint64_t rows0 = 0;  // rows of src[0] (a second source stacks below them)
};

struct Arena {
    uint8_t *base = nullptr;
    size_t bytes = 0;
    std::array<Piece, SLOT_COUNT> piece{};

    bool has(Slot s) const { return piece[s].on; }
    QW q(Slot s) const { return QW{piece[s].L, base + piece[s].off}; }
    float *f(Slot s) const { return reinterpret_cast<float *>(base + piece[s].off); }
};

// layer kinds (bits): every layer is DeltaNet or attention; some also take the n-gram embedding
enum : unsigned { K_MODEL = 1, K_MODEL_NG = 2, K_DELTA = 4, K_ATTN = 8, K_LAYER = K_DELTA | K_ATTN, K_NGRAM = 16 };

struct Layer : Arena {
    unsigned kind = 0;
    bool attn() const { return kind & K_ATTN; }
    bool ngram() const { return kind & K_NGRAM; }
};

// activations of one call (MAXT tokens), carved from one allocation
struct Acts {
    float *hb[2] = {}, *hn = nullptr, *lr = nullptr, *t320 = nullptr, *a = nullptr, *x = nullptr, *inj = nullptr;
    float *qkv = nullptr, *zz = nullptr, *abv = nullptr, *on = nullptr, *qg = nullptr, *kk = nullptr, *vv = nullptr;
    float *iqk = nullptr, *og = nullptr, *y = nullptr, *rsgv = nullptr, *shg = nullptr, *shu = nullptr;
    float *sha = nullptr, *shd = nullptr, *act = nullptr, *dpart = nullptr, *wsel = nullptr, *logits = nullptr;
    float *amv = nullptr, *work = nullptr;
    float *ng_emb = nullptr, *ng_key = nullptr, *ng_val = nullptr;
    int32_t *sel = nullptr, *pos = nullptr, *ami = nullptr, *ng_tok = nullptr;
    uint64_t *ng_tab = nullptr;  // n-gram hash: multipliers [3], then per head its table size, then its first row
    // one call's exchange with the host, one block so that a call needs one copy in and one out:
    // io = [MAXT token ids][status word][MAXT argmax ids]
    int32_t *io = nullptr, *ids = nullptr, *am = nullptr;
    unsigned *status = nullptr;  // the model's own misuse word (FN_STATUS_* bits of its attention kernels)
};

constexpr int AM_CH = 128;  // chunks of the two-pass argmax
constexpr int IO_WORDS = 2 * MAXT + 1;  // Acts::io
constexpr int HC_KS = 4;    // split of the hyper-connection down product along its rows (several-token calls)

struct Model {
    ModelDims d;
    int max_ctx = 0, nsplit = 1;
    Arena top;                  // model-wide tensors
    std::vector<Layer> layers;
    Acts a;
    size_t work_bytes = 0;
    hipStream_t st = nullptr;
    // the residual streams of the current stage and the other buffer of the pair a fused write moves them to
    float *h = nullptr, *h2 = nullptr;
    // pinned host staging of Acts::io (an asynchronous copy from or to pageable memory is a blocking one)
    int32_t *h_io = nullptr;
    void *host = nullptr;
    hipGraphExec_t graph[MAXT + 1] = {};
    bool use_graphs = true;
    bool failed = false;  // a call's kernels recorded misuse: device positions and state are not the host's
    float *dbg = nullptr;  // host [NL][nt][HC D] when set
    int n_past = 0;
    double last_ms = 0;
    std::vector<void *> allocs;
    size_t bytes = 0;

    Model() = default;
    Model(const Model &) = delete;
    Model &operator=(const Model &) = delete;
    ~Model();
};

// parse the shapes of a GGUF's model (<arch>.* metadata and the token table)
int read_dims(const Gguf &g, ModelDims &d);
// the arenas of the model of g (and its second shard g2, may be unmapped): every tensor found and checked, every
// piece's place known; no device work
int plan_weights(Model &m, const Gguf &g, const Gguf &g2);
// the planned arenas on the current device (weights, zeroed state), the n-gram hash and the activations of MAXT
// tokens; the mappings of the planned tensors must be alive, and are not needed afterwards
int commit_weights(Model &m);

// n-gram embedding (ngram.hip): a call of nt tokens at device position *pos; the conv input ring of a layer
// (NG_HIST) is NG_RING x HC D floats, the input of position p at slot p mod NG_RING
struct NgramCall {
    int nt = 0, HC = 0, D = 0;
    float eps = 0;
    const int32_t *pos = nullptr;
};
// the gated value of each stream and the dilated conv of its normalised form, added to the streams h [nt][HC D]:
// key [nt][HC D] and val [nt][D] are the key and value projections of the gathered rows (ngram.hip)
int ngram_inject_launch(const NgramCall &c, const float *key, const float *val, float *h, const Layer &L,
                        hipStream_t st);

}  // namespace fn
