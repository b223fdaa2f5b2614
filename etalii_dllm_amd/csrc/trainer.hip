// The device-resident fine-tuning step (include/dllm_hip.h, dllm_hip_trainer_*).
//
// Restates FineTuner.train_step (src/etalii_dllm/training/trainer.py:290-335), DecoderGradients
// (training/backprop.py:88-118, 183-377, 399-527) and AdamW.step (training/optimizer.py:82-109) for pre-norm
// decoders (Llama, Mistral, Qwen2, Qwen3 dense; Mixtral, OLMoE routed experts) on one GPU:
//  - all windows of a step are packed into one batch of rows. Row-local work (linear, dX, norms, RoPE, SwiGLU,
//    cross-entropy) is independent of the rows it is batched with, so packing changes no bit;
//  - every reduction over a window's rows (dW, db, norm weights, the embedding) is done per window and the per-window
//    float32 results are added in window order, the first copied (trainer.py:328-332), inside the kernels;
//  - the float32 glue of backprop.py is fused into the producing kernels with its operand order: x_mid = x + out and
//    x_out = x_mid + mlp in the projection epilogues, dh1 = (dq + dk) + dv and dh2 = dx_gate + dx_up in the dX
//    epilogues, dx_mid = dx + dh2' and dx = dx_mid + dh1' in the norm-backward kernels;
//  - the tied embedding's gradient (dembedding + dhead per window, then summed over windows) is the head dW with the
//    window's embedding rows as an addend;
//  - routed experts (backprop.py:308-357, 501-527): after each layer's routing the chosen experts come back to the
//    host, which groups the step's rows by expert (experts ascending, rows ascending: a window's group is a
//    contiguous run inside the step's group) and splits each group at the window boundaries, so an expert's dW is
//    the same per-window float sum as any other weight's. An expert no row of a window reaches adds that window's
//    +0.0f, as the reference's zero gradient does.
// Weights, gradients and AdamW moments live in one arena each, tensors in natural name order.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "attn_step.h"
#include "common.h"
#include "devmath.h"
#include "dllm_hip.h"
#include "export.h"
#include "kernels.h"

using namespace dllm_hip;

namespace {

// ---- natural name order (modelfile.py:40-47) ----
struct Part {
    bool digits;
    long long number;
    std::string text;
};

std::vector<Part> split_name(const std::string& name) {
    std::vector<Part> parts;
    size_t i = 0;
    std::string text;
    while (i <= name.size()) {
        if (i < name.size() && isdigit(static_cast<unsigned char>(name[i]))) {
            parts.push_back({false, 0, text});
            text.clear();
            size_t j = i;
            while (j < name.size() && isdigit(static_cast<unsigned char>(name[j]))) ++j;
            parts.push_back({true, std::strtoll(name.substr(i, j - i).c_str(), nullptr, 10), ""});
            i = j;
            continue;
        }
        if (i == name.size()) break;
        text.push_back(name[i]);
        ++i;
    }
    parts.push_back({false, 0, text});
    return parts;
}

bool natural_less(const std::string& a, const std::string& b) {
    const std::vector<Part> pa = split_name(a), pb = split_name(b);
    const size_t n = std::min(pa.size(), pb.size());
    for (size_t i = 0; i < n; ++i) {
        const Part &x = pa[i], &y = pb[i];
        if (x.digits != y.digits) return x.digits;  // (0, n, "") sorts before (1, 0, text)
        if (x.digits) {
            if (x.number != y.number) return x.number < y.number;
        } else if (x.text != y.text) {
            return x.text < y.text;
        }
    }
    if (pa.size() != pb.size()) return pa.size() < pb.size();
    return a < b;
}

// ---- device memory ----
struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t n) {
        bytes = n > 0 ? n : 1;
        return check_hip(hipMalloc(&p, bytes), "hipMalloc");
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

struct TensorInfo {
    std::string name;
    int64_t offset = 0, numel = 0, rows = 0, cols = 0;
    int ndim = 1;
    int64_t wt_offset = -1;  // transposed copy for the forward matmul, if it is a linear weight
};

// fold_scales (transformer.py:212-245): dst = src with every entry of row r times the float rowscale[r]; rows of
// `cols` elements (1 for vectors). The RoPE attention factor's table holds the factor on the rows feeding rotated
// dimensions ((r % head_dim) < rotary_dim) and 1 elsewhere (x * 1 is x); the residual multiplier's holds it on every
// row.
__global__ void fold_rows_kernel(const float* __restrict__ src, float* __restrict__ dst, int64_t n, int64_t cols,
                                 const float* __restrict__ rowscale) {
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; e < n;
         e += static_cast<int64_t>(gridDim.x) * 256)
        dst[e] = src[e] * rowscale[e / cols];
}

// rope_inv_freq (numerics.py:267-297, default scaling): exp(-(2i / dim) log(theta)) with the portable exp and log.
__global__ void inv_freq_kernel(int64_t rotary_dim, double theta, double* out) {
    const int64_t i = threadIdx.x + static_cast<int64_t>(blockIdx.x) * blockDim.x;
    if (i >= rotary_dim / 2) return;
    const double log_theta = dlog(theta);
    const double frac = static_cast<double>(2 * i) / static_cast<double>(rotary_dim);
    out[i] = dexp(-frac * log_theta);
}

// Untied embedding gradient: out[v][d] = window-ordered float sum of the windows' rows for token v (a window without
// token v contributes +0.0f), the first window copied.
__global__ __launch_bounds__(256) void sparse_window_sum_kernel(const float* __restrict__ rows,
                                                                const int* __restrict__ addrow, int64_t vocab,
                                                                int64_t dim, int windows,
                                                                const float* __restrict__ weights,
                                                                float* __restrict__ out) {
    const int64_t v = blockIdx.x;
    for (int64_t d = threadIdx.x; d < dim; d += 256) {
        float t = 0.0f;
        for (int w = 0; w < windows; ++w) {
            const int r = addrow[static_cast<int64_t>(w) * vocab + v];
            float val = r >= 0 ? rows[static_cast<int64_t>(r) * dim + d] : 0.0f;
            if (weights) val = val * weights[w];  // the window's whole gradient times its factor
            t = w == 0 ? val : t + val;
        }
        out[v * dim + d] = t;
    }
}

}  // namespace

struct dllm_hip_trainer {
    dllm_hip_decoder_config c{};
    int64_t R_max = 0, W_max = 0, T_max = 0;
    int64_t H = 0, QD = 0, KVD = 0, I = 0, V = 0;
    std::vector<TensorInfo> tensors;
    std::map<std::string, int> index;
    DevBuf params, grads, m1, m2, wt;

    struct LayerIds {
        int attn_norm, q, k, v, qb = -1, kb = -1, vb = -1, qn = -1, kn = -1, o, mlp_norm, gate, up, down;
        int router = -1;
        int attn_post = -1, mlp_post = -1;   // post norms (OLMo 2; sandwich with the pre norms)
        int sgate = -1, sup = -1, sdown = -1, sgw = -1;  // the shared expert and its gate (Qwen2-MoE)
        std::vector<int> egate, eup, edown;  // routed experts
    };
    std::vector<LayerIds> layer_ids;
    int emb = -1, final_norm = -1, lm_head = -1;

    struct Saved {
        float *x_in, *h1, *q_raw, *k_raw, *qn, *kn, *q, *k, *v, *attended, *x_mid, *h2, *gate, *up, *gate_act, *product;
        float *out = nullptr, *mlp = nullptr;  // post norms: the attention and MLP outputs before their norms
        // the shared expert over every row: gate/up/activation/product [R][SI], y [R][H], the gate's sigmoid [R]
        float *sh_gate = nullptr, *sh_up = nullptr, *sh_act = nullptr, *sh_product = nullptr, *sh_y = nullptr,
              *sh_s = nullptr;
        // routed experts: router logits and probabilities [R][E], the choices [R][K] (rank order), the expert
        // outputs y [R K][H] in grouped order (gate, up, gate_act, product are grouped [R K][EI] then)
        float *router_logits = nullptr, *probs = nullptr, *routing = nullptr, *y = nullptr;
        int64_t* chosen = nullptr;
        // grouping: position p of the grouped rows holds row row_of[p], routing slot slot[p]; order[r K + i] is the
        // position of row r's i-th choice by ascending expert; eseg[e][w] the window boundaries in expert e's group
        int64_t *row_of = nullptr, *slot = nullptr, *order = nullptr, *eseg = nullptr;
        std::vector<int64_t> estart;  // host: E + 1 group starts
        // the layer's expert matmuls, one grouped launch per kind (tables in device memory, made by group_rows)
        GemmGroup groups[9];
        double group_flops[9] = {};
        // a kind whose matmuls the grouped kernel cannot stage (sizes not whole 16-byte chunks): one launch each
        std::vector<GemmCall> loose[9];
        // grouping on the device: the group starts [E + 1] and each kind's template table (gemm_row_group_prepare),
        // valid for the step shape in tmpl_key
        int64_t* estart_d = nullptr;
        char* tmpl = nullptr;
        std::vector<int64_t> tmpl_key;
        char* tables = nullptr;
    };
    enum ExpertMatmul { kFwdGate, kFwdUp, kFwdDown, kDxDown, kDwDown, kDxGate, kDwGate, kDxUp, kDwUp, kExpertMatmuls };
    std::vector<Saved> saved;
    std::vector<std::unique_ptr<DevBuf>> owned;
    float *x_final = nullptr, *hidden = nullptr, *logits = nullptr, *dlogits = nullptr;
    float* logits_capped = nullptr;  // Gemma 2's soft-capped logits (the uncapped ones stay in `logits`)
    float *dx = nullptr, *dh = nullptr, *dx_mid = nullptr, *dattended = nullptr, *dq_t = nullptr, *dk_t = nullptr,
          *dv_t = nullptr, *dq = nullptr, *dk = nullptr, *dq2 = nullptr, *dk2 = nullptr, *dproduct = nullptr,
          *dgate = nullptr, *dup = nullptr, *col_part = nullptr, *col_part_side = nullptr, *emb_rows = nullptr,
          *gemm_part = nullptr;
    int64_t gemm_part_cap = 0;  // floats: per-window partials of the layer weight gradients
    // routed experts: E experts, K per token, EI expert intermediate size; shared buffers of the grouped rows
    int64_t E = 0, K = 0, EI = 0, RK = 0;
    float *xg = nullptr, *dyg = nullptr, *dxg = nullptr, *dweights = nullptr, *dlogits_r = nullptr, *dprob = nullptr,
          *dh2r = nullptr, *grad_row = nullptr;
    double* router_loss_w = nullptr;
    float* probs_all = nullptr;
    int64_t* counts_d = nullptr;
    int64_t* pos_of = nullptr;     // grouping scratch [R K]: each choice's grouped position
    void* group_cnt = nullptr;     // grouping scratch [W][E] 8-byte counters
    int* route_err = nullptr;      // set by the grouping for an expert out of range
    int64_t tmpl_version = 0;      // bumped when the step's weight addresses change (fold, merge)
    std::vector<int64_t> counts_host;  // [windows][E] choices per window over all layers
    double router_scale_cur = 0.0, last_router_loss = 0.0;
    double *inv_mlp = nullptr, *inv_attn = nullptr, *inv_post = nullptr;
    float *post_tmp = nullptr, *dpost = nullptr;
    // shared experts: the gated output term and the MLP output [R][H]; the backward's dy, dx [R][H], its dproduct,
    // dgate, dup [R][SI], the gate score's gradient [R] and the gate dW's per-window partial sums [W][H]
    float *sh_term = nullptr, *sh_out = nullptr, *dsh_dy = nullptr, *dsh_x = nullptr, *dsh_product = nullptr,
          *dsh_gate = nullptr, *dsh_up = nullptr, *dsh_score = nullptr, *sh_part = nullptr;  // post norms: a normalised block output; a norm's input gradient  // the layer norms' inverse rms, read by their weights' gradients
    double *inv_rms = nullptr, *row_max = nullptr, *row_total = nullptr, *row_loss = nullptr, *loss_w = nullptr,
           *stats = nullptr, *inv_freq = nullptr, *cos_t = nullptr, *sin_t = nullptr;
    // Gemma 3's windowed layers rotate with a base of their own and no scaling (backprop.py:63-67)
    double *inv_local = nullptr, *cos_local = nullptr, *sin_local = nullptr;
    void* attn_ws = nullptr;
    int64_t *tok_in = nullptr, *tok_tgt = nullptr, *pos_index = nullptr, *seg_d = nullptr, *batch_d = nullptr,
            *grp_order = nullptr, *grp_start = nullptr, *grp_out = nullptr;
    int* addrow = nullptr;
    int* err_flag = nullptr;
    std::vector<int64_t> seg_host;
    bool wt_valid = false;
    // per-layer choices (dense_layers, full_attention_layers): from the config's flag arrays, or its 64-bit masks
    std::vector<char> dense_flag, full_flag;
    // Model sizes that are not whole 16-byte chunks (a vocabulary of 50257, an intermediate size of 30): the matmuls
    // whose operands cannot be staged by the matrix-core kernel widen their A operand into this double scratch and
    // run on the VALU kernels (same per-output chains, same bits). One scratch, so such steps keep to one stream.
    bool odd_shapes = false;
    double* mm_scratch = nullptr;
    int64_t mm_scratch_cap = 0;

    // What AdamW updates: parameters, gradients and moments of one set of tensors in one arena each, the chunk table
    // of the fused update and the plan of the exact global norm (optimizer.py:66-109).
    struct OptimizerSet {
        float *p = nullptr, *g = nullptr, *m = nullptr, *v = nullptr;
        int64_t tensors = 0, chunks = 0;
        int64_t *chunk_start = nullptr, *chunk_end = nullptr;
        double *chunk_decay = nullptr, *chunk_decay_scaled = nullptr, *per_tensor = nullptr;
        double last_decay = -1.0;
        ExactSumPlan norm_plan;
        void* norm_ws = nullptr;
    };
    OptimizerSet main_opt, lora_opt;

    // LoRA runs (lora.py): adapters in natural name order in their own arenas, the merged weights the step uses for
    // the targets, and (Q8_0 base) the quantisable matrices held as their dequantised values.
    bool lora_on = false;
    dllm_hip_lora_config lc{};
    float lora_scale = 0.0f;
    std::vector<TensorInfo> adapters;
    std::map<std::string, int> adapter_index;
    struct LoraTarget {
        int weight, a, b;  // tensor id, adapter ids
    };
    std::vector<LoraTarget> lora_targets;
    // LoRA runs compute the gradients of the adapted weights only: the others reach no optimizer (trainer.py:463-474)
    std::vector<const float*> target_grads;
    bool grad_wanted(const float* g) const {
        return !lora_on || std::find(target_grads.begin(), target_grads.end(), g) != target_grads.end();
    }
    DevBuf lora_p, lora_g, lora_m, lora_v, merged;
    std::vector<int64_t> merged_offset;  // per tensor id: offset in `merged`, or -1
    // fold_scales (transformer.py:224-245): the step reads the q/k rows feeding the rotated dimensions (or the QK-norm
    // entries) times the LongRoPE / YaRN attention factor, and the output and down projections times Granite's
    // residual multiplier, from `folded`; each window's gradients of those tensors are multiplied by the same factors
    // (_unfold, backprop.py:380-394) before the window sum.
    bool fold_on = false;
    double rope_factor = 1.0;
    DevBuf folded;
    std::vector<int64_t> fold_offset;      // per tensor id: offset in `folded`, or -1
    std::vector<const float*> fold_table;  // per tensor id: its per-row factors, or null
    float* rope_rowscale = nullptr;        // [q heads x head_dim]: the factor on rotated entries, 1 elsewhere
    float* resid_rowscale = nullptr;       // [hidden]: the residual multiplier
    bool base_ready = true;              // the Q8_0 base has been applied to the current parameters
    void* lora_ws = nullptr;
    size_t lora_ws_bytes = 0;
    int8_t* q8_values = nullptr;
    float* q8_scales = nullptr;
    uint8_t* q4_packed = nullptr;  // a Q4_0 base: the packed values before unpacking
    char* staging = nullptr;       // pinned host memory: a step's inputs on their way to the device
    size_t staging_bytes = 0;
    // attention as batched matmuls (attn_lds.hip, attn_chains.hip): per (window, head) transposed operands and score
    // matrices
    int64_t Tp = 0;
    double* attn_dvec = nullptr;  // the softmax backward's per-query D
    double* attn_slope = nullptr;
    double *attn_et = nullptr, *attn_inv = nullptr, *attn_dpt = nullptr, *attn_pg = nullptr, *attn_dsg = nullptr;
    double* attn_tmax = nullptr;  // the scores' per-64-key-tile maxima of each query [z][Tp / 64][Tp]
    float *attn_qt = nullptr, *attn_dot = nullptr;

    template <typename T>
    int make(T** out, size_t n) {
        owned.emplace_back(new DevBuf());
        DLLM_TRY(owned.back()->alloc(n * sizeof(T)));
        *out = owned.back()->as<T>();
        return kOk;
    }

    int add_tensor(const std::string& name, int64_t rows, int64_t cols, bool linear_weight) {
        TensorInfo t;
        t.name = name;
        t.rows = rows;
        t.cols = cols;
        t.ndim = cols > 0 ? 2 : 1;
        t.numel = cols > 0 ? rows * cols : rows;
        t.wt_offset = linear_weight ? 0 : -1;
        tensors.push_back(t);
        return kOk;
    }

    // Whether layer l's MLP is a mixture of experts (TransformerConfig.is_sparse, architecture.py:344-346): every
    // layer of a model with experts except those in dense_layers.
    bool sparse(int64_t l) const { return E > 0 && !dense_flag[static_cast<size_t>(l)]; }
    // Norm placement (architecture.py:315-320): pre (each block's input), post (its output; OLMo 2) or both.
    bool pre_norms() const { return c.norm_placement != 1; }
    int uo() const { return c.norm_unit_offset ? 1 : 0; }  // norms with 1 + w (Gemma)
    int act() const { return static_cast<int>(c.activation); }
    // TransformerConfig.window (architecture.py:353-359): the sliding window of layer l, 0 for full attention
    int64_t layer_window(int64_t l) const {
        if (c.sliding_window == 0) return 0;
        return full_flag[static_cast<size_t>(l)] ? 0 : c.sliding_window;
    }
    // The RoPE tables of layer l (uses_local_rope, architecture.py:322-324)
    bool local_rope(int64_t l) const { return c.local_rope_theta != 0.0 && layer_window(l) != 0; }
    const double* cos_of(int64_t l) const { return local_rope(l) ? cos_local : cos_t; }
    const double* sin_of(int64_t l) const { return local_rope(l) ? sin_local : sin_t; }
    bool post_norms() const { return c.norm_placement != 0; }
    int64_t sparse_layers() const {
        int64_t n = 0;
        for (int64_t l = 0; l < c.layers; ++l) n += sparse(l) ? 1 : 0;
        return n;
    }

    int build_tensors() {
        const auto& k = c;
        add_tensor("token_embedding.weight", V, H, k.tie_embeddings != 0);
        for (int64_t l = 0; l < k.layers; ++l) {
            const std::string p = "layers." + std::to_string(l) + ".";
            if (pre_norms()) add_tensor(p + "attention_norm.weight", H, 0, false);
            add_tensor(p + "attention.q.weight", QD, H, true);
            add_tensor(p + "attention.k.weight", KVD, H, true);
            add_tensor(p + "attention.v.weight", KVD, H, true);
            if (k.attention_bias) {
                add_tensor(p + "attention.q.bias", QD, 0, false);
                add_tensor(p + "attention.k.bias", KVD, 0, false);
                add_tensor(p + "attention.v.bias", KVD, 0, false);
            }
            if (k.qk_norm) {
                add_tensor(p + "attention.q_norm.weight", k.qk_norm == 2 ? QD : k.head_dim, 0, false);
                add_tensor(p + "attention.k_norm.weight", k.qk_norm == 2 ? KVD : k.head_dim, 0, false);
            }
            add_tensor(p + "attention.o.weight", H, QD, true);
            if (post_norms()) {
                add_tensor(p + "attention_post_norm.weight", H, 0, false);
                add_tensor(p + "mlp_post_norm.weight", H, 0, false);
            }
            if (pre_norms()) add_tensor(p + "mlp_norm.weight", H, 0, false);
            if (sparse(l)) {  // architecture.py: a routed layer has the router and E experts instead of the dense MLP
                add_tensor(p + "mlp.router.weight", E, H, true);
                for (int64_t e = 0; e < E; ++e) {
                    const std::string x = p + "mlp.experts." + std::to_string(e) + ".";
                    add_tensor(x + "gate.weight", EI, H, true);
                    add_tensor(x + "up.weight", EI, H, true);
                    add_tensor(x + "down.weight", H, EI, true);
                }
                if (k.shared_inter > 0) {
                    add_tensor(p + "mlp.shared.gate.weight", k.shared_inter, H, true);
                    add_tensor(p + "mlp.shared.up.weight", k.shared_inter, H, true);
                    add_tensor(p + "mlp.shared.down.weight", H, k.shared_inter, true);
                    if (k.shared_gate) add_tensor(p + "mlp.shared_gate.weight", 1, H, false);
                }
            } else {
                add_tensor(p + "mlp.gate.weight", I, H, true);
                add_tensor(p + "mlp.up.weight", I, H, true);
                add_tensor(p + "mlp.down.weight", H, I, true);
            }
        }
        add_tensor("final_norm.weight", H, 0, false);
        if (!k.tie_embeddings) add_tensor("lm_head.weight", V, H, true);
        std::stable_sort(tensors.begin(), tensors.end(),
                         [](const TensorInfo& a, const TensorInfo& b) { return natural_less(a.name, b.name); });
        int64_t off = 0, wt_off = 0;
        for (size_t i = 0; i < tensors.size(); ++i) {
            TensorInfo& t = tensors[i];
            off = static_cast<int64_t>(round_up(static_cast<size_t>(off), 64));  // 256-byte aligned tensors
            t.offset = off;
            off += t.numel;
            if (t.wt_offset >= 0) {
                wt_off = static_cast<int64_t>(round_up(static_cast<size_t>(wt_off), 64));
                t.wt_offset = wt_off;
                wt_off += t.numel;
            }
            index[t.name] = static_cast<int>(i);
        }
        const size_t arena = static_cast<size_t>(round_up(static_cast<size_t>(off), 64)) * sizeof(float);
        DLLM_TRY(params.alloc(arena));
        DLLM_TRY(grads.alloc(arena));
        DLLM_TRY(m1.alloc(arena));
        DLLM_TRY(m2.alloc(arena));
        DLLM_TRY(wt.alloc(static_cast<size_t>(wt_off > 0 ? wt_off : 1) * sizeof(float)));
        DLLM_TRY(check_hip(hipMemset(params.p, 0, arena), "memset"));
        DLLM_TRY(check_hip(hipMemset(grads.p, 0, arena), "memset"));
        DLLM_TRY(check_hip(hipMemset(m1.p, 0, arena), "memset"));
        DLLM_TRY(check_hip(hipMemset(m2.p, 0, arena), "memset"));
        auto id = [&](const std::string& n) { return index.count(n) ? index[n] : -1; };
        emb = id("token_embedding.weight");
        final_norm = id("final_norm.weight");
        lm_head = id("lm_head.weight");
        for (int64_t l = 0; l < c.layers; ++l) {
            const std::string p = "layers." + std::to_string(l) + ".";
            LayerIds L;
            L.attn_norm = id(p + "attention_norm.weight");
            L.q = id(p + "attention.q.weight");
            L.k = id(p + "attention.k.weight");
            L.v = id(p + "attention.v.weight");
            L.qb = id(p + "attention.q.bias");
            L.kb = id(p + "attention.k.bias");
            L.vb = id(p + "attention.v.bias");
            L.qn = id(p + "attention.q_norm.weight");
            L.kn = id(p + "attention.k_norm.weight");
            L.o = id(p + "attention.o.weight");
            L.mlp_norm = id(p + "mlp_norm.weight");
            L.attn_post = id(p + "attention_post_norm.weight");
            L.sgate = id(p + "mlp.shared.gate.weight");
            L.sup = id(p + "mlp.shared.up.weight");
            L.sdown = id(p + "mlp.shared.down.weight");
            L.sgw = id(p + "mlp.shared_gate.weight");
            L.mlp_post = id(p + "mlp_post_norm.weight");
            L.gate = id(p + "mlp.gate.weight");
            L.up = id(p + "mlp.up.weight");
            L.down = id(p + "mlp.down.weight");
            L.router = id(p + "mlp.router.weight");
            for (int64_t e = 0; e < E; ++e) {
                const std::string x = p + "mlp.experts." + std::to_string(e) + ".";
                L.egate.push_back(id(x + "gate.weight"));
                L.eup.push_back(id(x + "up.weight"));
                L.edown.push_back(id(x + "down.weight"));
            }
            layer_ids.push_back(L);
        }
        merged_offset.assign(tensors.size(), -1);
        DLLM_TRY(make(&stats, 3));
        return build_optimizer(tensors, params.as<float>(), grads.as<float>(), m1.as<float>(), m2.as<float>(),
                               &main_opt);
    }

    // AdamW chunk table (64K-element chunks inside each tensor, decay for matrices: optimizer.py:93) and the exact
    // parallel global-norm plan (sumsq.hip) over one arena's tensors.
    int build_optimizer(const std::vector<TensorInfo>& ts, float* p, float* g, float* m, float* v, OptimizerSet* o) {
        o->p = p;
        o->g = g;
        o->m = m;
        o->v = v;
        std::vector<int64_t> cs, ce, to, tc;
        std::vector<double> cd;
        for (const TensorInfo& t : ts) {
            to.push_back(t.offset);
            tc.push_back(t.numel);
            for (int64_t st = 0; st < t.numel; st += 65536) {
                cs.push_back(t.offset + st);
                ce.push_back(t.offset + std::min<int64_t>(t.numel, st + 65536));
                cd.push_back(t.ndim >= 2 ? 1.0 : 0.0);
            }
        }
        o->tensors = static_cast<int64_t>(ts.size());
        o->chunks = static_cast<int64_t>(cs.size());
        DLLM_TRY(make(&o->chunk_start, std::max<size_t>(cs.size(), 1)));
        DLLM_TRY(make(&o->chunk_end, std::max<size_t>(ce.size(), 1)));
        DLLM_TRY(make(&o->chunk_decay, std::max<size_t>(cd.size(), 1)));
        DLLM_TRY(make(&o->chunk_decay_scaled, std::max<size_t>(cd.size(), 1)));
        DLLM_TRY(check_hip(hipMemcpy(o->chunk_start, cs.data(), cs.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(check_hip(hipMemcpy(o->chunk_end, ce.data(), ce.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(check_hip(hipMemcpy(o->chunk_decay, cd.data(), cd.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(make(&o->per_tensor, std::max<size_t>(ts.size(), 1)));
        const size_t nb = exact_sum_squares_blocks(tc.data(), static_cast<int64_t>(tc.size()));
        std::vector<int64_t> tf(tc.size()), tb(tc.size()), bs(nb), bc(nb);
        exact_sum_squares_plan(to.data(), tc.data(), static_cast<int64_t>(tc.size()), tf.data(), tb.data(), bs.data(),
                               bc.data());
        int64_t *d_tf, *d_tb, *d_bs, *d_bc;
        DLLM_TRY(make(&d_tf, std::max<size_t>(tf.size(), 1)));
        DLLM_TRY(make(&d_tb, std::max<size_t>(tb.size(), 1)));
        DLLM_TRY(make(&d_bs, std::max<size_t>(bs.size(), 1)));
        DLLM_TRY(make(&d_bc, std::max<size_t>(bc.size(), 1)));
        DLLM_TRY(check_hip(hipMemcpy(d_tf, tf.data(), tf.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(check_hip(hipMemcpy(d_tb, tb.data(), tb.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(check_hip(hipMemcpy(d_bs, bs.data(), bs.size() * 8, hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(check_hip(hipMemcpy(d_bc, bc.data(), bc.size() * 8, hipMemcpyHostToDevice), "upload"));
        o->norm_plan.tensors = static_cast<int64_t>(tc.size());
        o->norm_plan.blocks = static_cast<int64_t>(nb);
        o->norm_plan.tfirst = d_tf;
        o->norm_plan.tblocks = d_tb;
        o->norm_plan.bstart = d_bs;
        o->norm_plan.bcount = d_bc;
        char* ws = nullptr;
        DLLM_TRY(make(&ws, exact_sum_squares_workspace(nb)));
        o->norm_ws = ws;
        return kOk;
    }

    int build_activations() {
        const int64_t R = R_max, heads = c.heads, kvh = c.kv_heads;
        saved.resize(static_cast<size_t>(c.layers));
        // [sparse layer][row][expert], the router statistics' input
        if (E > 0) DLLM_TRY(make(&probs_all, std::max<int64_t>(sparse_layers(), 1) * R * E));
        // x_in of layer l + 1 is x_out of layer l: one chain of L + 1 residual buffers.
        std::vector<float*> xs(static_cast<size_t>(c.layers) + 1);
        for (auto& p : xs) DLLM_TRY(make(&p, R * H));
        for (int64_t l = 0, routed = 0; l < c.layers; ++l) {
            Saved& s = saved[static_cast<size_t>(l)];
            s.x_in = xs[static_cast<size_t>(l)];
            if (pre_norms()) DLLM_TRY(make(&s.h1, R * H));
            else s.h1 = s.x_in;  // without pre norms the blocks read the residual stream itself
            DLLM_TRY(make(&s.q_raw, R * QD));
            DLLM_TRY(make(&s.k_raw, R * KVD));
            s.qn = s.kn = nullptr;
            if (c.qk_norm) {
                DLLM_TRY(make(&s.qn, R * QD));
                DLLM_TRY(make(&s.kn, R * KVD));
            }
            DLLM_TRY(make(&s.q, R * QD));
            DLLM_TRY(make(&s.k, R * KVD));
            DLLM_TRY(make(&s.v, R * KVD));
            DLLM_TRY(make(&s.attended, R * QD));
            DLLM_TRY(make(&s.x_mid, R * H));
            if (pre_norms()) DLLM_TRY(make(&s.h2, R * H));
            else s.h2 = s.x_mid;
            if (post_norms()) {
                DLLM_TRY(make(&s.out, R * H));
                DLLM_TRY(make(&s.mlp, R * H));
            }
            const int64_t mlp_rows = sparse(l) ? RK : R, mlp_inter = sparse(l) ? EI : I;
            DLLM_TRY(make(&s.gate, mlp_rows * mlp_inter));
            DLLM_TRY(make(&s.up, mlp_rows * mlp_inter));
            DLLM_TRY(make(&s.gate_act, mlp_rows * mlp_inter));
            DLLM_TRY(make(&s.product, mlp_rows * mlp_inter));
            if (sparse(l)) {
                DLLM_TRY(make(&s.router_logits, R * E));
                s.probs = probs_all + (routed++) * R * E;
                DLLM_TRY(make(&s.routing, RK));
                DLLM_TRY(make(&s.y, RK * H));
                DLLM_TRY(make(&s.chosen, RK));
                DLLM_TRY(make(&s.row_of, RK));
                DLLM_TRY(make(&s.slot, RK));
                DLLM_TRY(make(&s.order, RK));
                DLLM_TRY(make(&s.eseg, E * (W_max + 1)));
                DLLM_TRY(make(&s.tables, kExpertMatmuls * gemm_group_bytes(static_cast<int>(E))));
                DLLM_TRY(make(&s.tmpl, kExpertMatmuls * gemm_group_bytes(static_cast<int>(E))));
                DLLM_TRY(make(&s.estart_d, E + 1));
                if (c.shared_inter > 0) {
                    const int64_t SI = c.shared_inter;
                    DLLM_TRY(make(&s.sh_gate, R * SI));
                    DLLM_TRY(make(&s.sh_up, R * SI));
                    DLLM_TRY(make(&s.sh_act, R * SI));
                    DLLM_TRY(make(&s.sh_product, R * SI));
                    DLLM_TRY(make(&s.sh_y, R * H));
                    DLLM_TRY(make(&s.sh_s, R));
                }
            }
        }
        if (E > 0 && c.shared_inter > 0) {
            const int64_t SI = c.shared_inter;
            for (float** b : {&sh_term, &sh_out, &dsh_dy, &dsh_x}) DLLM_TRY(make(b, R * H));
            for (float** b : {&dsh_product, &dsh_gate, &dsh_up}) DLLM_TRY(make(b, R * SI));
            DLLM_TRY(make(&dsh_score, R));
            DLLM_TRY(make(&sh_part, W_max * H));
        }
        if (E > 0) {
            DLLM_TRY(make(&xg, RK * H));
            DLLM_TRY(make(&dyg, RK * H));
            DLLM_TRY(make(&dxg, RK * H));
            DLLM_TRY(make(&dweights, RK));
            DLLM_TRY(make(&dlogits_r, R * E));
            DLLM_TRY(make(&dprob, R * E));
            DLLM_TRY(make(&dh2r, R * H));
            DLLM_TRY(make(&grad_row, W_max * E));
            DLLM_TRY(make(&router_loss_w, W_max));
            DLLM_TRY(make(&counts_d, W_max * E));
            DLLM_TRY(make(&pos_of, RK));
            char* gc = nullptr;
            DLLM_TRY(make(&gc, static_cast<size_t>(W_max * E) * 8));
            group_cnt = gc;
            DLLM_TRY(make(&route_err, 1));
        }
        const int64_t dmlp = std::max(R * I, RK * EI);
        x_final = xs.back();
        DLLM_TRY(make(&hidden, R * H));
        DLLM_TRY(make(&logits, R * V));
        DLLM_TRY(make(&dlogits, R * V));
        DLLM_TRY(make(&dx, R * H));
        DLLM_TRY(make(&dh, R * H));
        DLLM_TRY(make(&dh_b, R * H));
        DLLM_TRY(make(&dh_c, R * H));
        DLLM_TRY(make(&dx_mid, R * H));
        DLLM_TRY(make(&dattended, R * QD));
        DLLM_TRY(make(&dq_t, R * QD));
        DLLM_TRY(make(&dk_t, R * KVD));
        DLLM_TRY(make(&dv_t, R * KVD));
        DLLM_TRY(make(&dq, R * QD));
        DLLM_TRY(make(&dk, R * KVD));
        DLLM_TRY(make(&dq2, R * QD));
        DLLM_TRY(make(&dk2, R * KVD));
        DLLM_TRY(make(&dproduct, dmlp));
        DLLM_TRY(make(&dgate, dmlp));
        DLLM_TRY(make(&dup, dmlp));
        DLLM_TRY(make(&col_part, W_max * std::max<int64_t>({H, QD, KVD, I})));
        DLLM_TRY(make(&col_part_side, W_max * std::max<int64_t>({H, QD, KVD})));
        if (W_max > 1) {
            gemm_part_cap = W_max * H * std::max<int64_t>({QD, KVD, I, EI, E});
            DLLM_TRY(make(&gemm_part, gemm_part_cap));
        }
        DLLM_TRY(make(&emb_rows, R * H));
        DLLM_TRY(make(&inv_rms, R * std::max<int64_t>(heads, 1)));
        DLLM_TRY(make(&inv_mlp, R));
        DLLM_TRY(make(&inv_attn, R));
        if (post_norms()) {
            DLLM_TRY(make(&inv_post, R));
            DLLM_TRY(make(&post_tmp, R * H));
            DLLM_TRY(make(&dpost, R * H));
        }
        DLLM_TRY(make(&dh1, R * H));
        DLLM_TRY(make(&row_max, R));
        DLLM_TRY(make(&row_total, R));
        DLLM_TRY(make(&row_loss, R));
        DLLM_TRY(make(&loss_w, W_max));
        DLLM_TRY(make(&win_weight, W_max));
        DLLM_TRY(make(&inv_freq, std::max<int64_t>(c.rotary_dim / 2, 1)));
        DLLM_TRY(make(&cos_t, T_max * std::max<int64_t>(c.rotary_dim / 2, 1)));
        DLLM_TRY(make(&sin_t, T_max * std::max<int64_t>(c.rotary_dim / 2, 1)));
        Tp = padded_rows(T_max);
        const int64_t hd = c.head_dim, G = heads / kvh;
        DLLM_TRY(make(&attn_qt, W_max * heads * hd * Tp));
        DLLM_TRY(make(&attn_dot, W_max * heads * hd * Tp));
        {
            // the saved attention numerators, and with soft-capped scores their 1 - tanh^2 factors: layers x windows x
            // heads x Tp^2 doubles each (quadratic in the window length), refused up front with the formula rather
            // than failing in the allocator
            const double saved_bytes = static_cast<double>(c.layers) * W_max * heads * Tp * Tp * 8.0 *
                                       (c.attention_softcap != 0.0 ? 2.0 : 1.0);
            size_t free_bytes = 0, total_bytes = 0;
            DLLM_TRY(check_hip(hipMemGetInfo(&free_bytes, &total_bytes), "hipMemGetInfo"));
            if (saved_bytes > static_cast<double>(free_bytes))
                return fail(kOutOfMemory,
                            "the saved attention scores need layers x max_windows x heads x Tp^2 x 8 bytes (Tp = "
                            "max_window_tokens rounded up to 64; twice that with attention_softcap): " +
                                std::to_string(saved_bytes / 1e9) + " GB, more than the " +
                                std::to_string(static_cast<double>(free_bytes) / 1e9) + " GB free");
        }
        DLLM_TRY(make(&attn_et, c.layers * W_max * heads * Tp * Tp));  // E^T saved per layer for the backward
        // soft-capped scores: the backward's factor 1 - tanh^2 of every score, saved per layer
        if (c.attention_softcap != 0.0) DLLM_TRY(make(&attn_slope, c.layers * W_max * heads * Tp * Tp));
        DLLM_TRY(make(&attn_inv, c.layers * W_max * heads * Tp));
        DLLM_TRY(make(&attn_dpt, W_max * heads * Tp * Tp));
        DLLM_TRY(make(&attn_pg, W_max * kvh * Tp * G * Tp));
        DLLM_TRY(make(&attn_dsg, W_max * kvh * Tp * G * Tp));
        DLLM_TRY(make(&attn_dvec, W_max * heads * Tp));
        DLLM_TRY(make(&attn_tmax, W_max * heads * (Tp / 64) * Tp));
        DLLM_TRY(make(&tok_in, R));
        DLLM_TRY(make(&tok_tgt, R));
        DLLM_TRY(make(&pos_index, R));
        DLLM_TRY(make(&seg_d, W_max + 1));
        DLLM_TRY(make(&batch_d, 4 * W_max));
        DLLM_TRY(make(&grp_order, R));
        DLLM_TRY(make(&grp_start, R + 1));
        DLLM_TRY(make(&grp_out, R));
        DLLM_TRY(make(&addrow, W_max * V));
        DLLM_TRY(make(&err_flag, 1));
        staging_bytes = static_cast<size_t>(8 * (7 * R_max + 5 * W_max + 8) + 4 * W_max * V) + 9 * 256;
        DLLM_TRY(check_hip(hipHostMalloc(reinterpret_cast<void**>(&staging), staging_bytes, hipHostMallocDefault),
                           "pinned staging"));
        // RoPE tables for positions 0 .. T_max - 1 (every window starts at position 0)
        hipLaunchKernelGGL(inv_freq_kernel, dim3(1), dim3(1024), 0, nullptr, c.rotary_dim, c.rope_theta, inv_freq);
        DLLM_TRY(check_launch("inv_freq"));
        DLLM_TRY(launch_rope_tables(nullptr, T_max, inv_freq, c.rotary_dim / 2, cos_t, sin_t, nullptr));
        if (c.local_rope_theta != 0.0) {
            DLLM_TRY(make(&inv_local, std::max<int64_t>(c.rotary_dim / 2, 1)));
            DLLM_TRY(make(&cos_local, T_max * std::max<int64_t>(c.rotary_dim / 2, 1)));
            DLLM_TRY(make(&sin_local, T_max * std::max<int64_t>(c.rotary_dim / 2, 1)));
            hipLaunchKernelGGL(inv_freq_kernel, dim3(1), dim3(1024), 0, nullptr, c.rotary_dim, c.local_rope_theta,
                               inv_local);
            DLLM_TRY(check_launch("inv_freq"));
            DLLM_TRY(launch_rope_tables(nullptr, T_max, inv_local, c.rotary_dim / 2, cos_local, sin_local, nullptr));
        }
        if (c.logits_softcap != 0.0) DLLM_TRY(make(&logits_capped, R * V));
        // the matmul scratch of sizes that are not whole 16-byte chunks: the widest A operand is [l][i] with
        // l x i = (a model size) x (the rows) either way round, i padded to whole row tiles
        const int64_t SI = c.shared_inter;
        for (int64_t d : {V, H, I, EI, E, SI}) odd_shapes = odd_shapes || d % 4 != 0;
        if (odd_shapes) {
            const int64_t widest = std::max<int64_t>({V, H, QD, KVD, I, EI, E, SI});
            mm_scratch_cap = std::max(widest * padded_rows(R), R * padded_rows(widest));
            DLLM_TRY(make(&mm_scratch, static_cast<size_t>(mm_scratch_cap)));
        }
        return check_hip(hipDeviceSynchronize(), "trainer setup");
    }

    // The weight as the stored model holds it (LoRA targets: merged)
    float* Psrc(int id) const {
        const int64_t mo = merged_offset.empty() ? -1 : merged_offset[static_cast<size_t>(id)];
        return mo >= 0 ? merged.as<float>() + mo : params.as<float>() + tensors[static_cast<size_t>(id)].offset;
    }
    // The weight as the step uses it (fold_scales applied)
    float* P(int id) const {
        const int64_t fo = fold_offset.empty() ? -1 : fold_offset[static_cast<size_t>(id)];
        return fo >= 0 ? folded.as<float>() + fo : Psrc(id);
    }
    // The per-row factors of a tensor's window gradients (the unfold), or null
    const float* unfold_scale(int id) const {
        return id >= 0 && !fold_table.empty() ? fold_table[static_cast<size_t>(id)] : nullptr;
    }

    // The folded copies of the scaled tensors from their current values.
    int fold_weights(hipStream_t s) {
        for (size_t i = 0; i < tensors.size(); ++i) {
            if (fold_offset[i] < 0) continue;
            const TensorInfo& t = tensors[i];
            const int64_t cols = t.cols > 0 ? t.cols : 1;
            const unsigned blocks = static_cast<unsigned>(std::min<int64_t>(ceil_div(t.numel, 256), 4096));
            hipLaunchKernelGGL(fold_rows_kernel, dim3(blocks), dim3(256), 0, s, Psrc(static_cast<int>(i)),
                               folded.as<float>() + fold_offset[i], t.numel, cols, fold_table[i]);
            DLLM_TRY(check_launch("fold"));
        }
        return kOk;
    }

    bool residual_on() const { return c.residual_multiplier != 1.0; }

    // Which tensors are folded and by which row factors: the rope-scaled ones (rope_scaled_tensors,
    // transformer.py:204-209: the QK-norm weights, else the q/k projections and biases) when the attention factor is
    // not 1, the "attention.o.weight" and "down.weight" tensors (every expert's) when the residual multiplier is not
    // 1. The sets are disjoint.
    int setup_fold() {
        const bool rope = rope_factor != 1.0, resid = residual_on();
        fold_offset.assign(tensors.size(), -1);
        fold_table.assign(tensors.size(), nullptr);
        int64_t off = 0;
        auto add = [&](int id, const float* table) {
            if (id < 0) return;
            fold_offset[static_cast<size_t>(id)] = off;
            fold_table[static_cast<size_t>(id)] = table;
            off += static_cast<int64_t>(round_up(static_cast<size_t>(tensors[static_cast<size_t>(id)].numel), 64));
        };
        for (const LayerIds& L : layer_ids) {
            if (rope) {
                const int ids[4] = {c.qk_norm ? L.qn : L.q, c.qk_norm ? L.kn : L.k, c.qk_norm ? -1 : L.qb,
                                    c.qk_norm ? -1 : L.kb};
                for (int id : ids) add(id, rope_rowscale);
            }
            if (resid) {
                add(L.o, resid_rowscale);
                add(L.down, resid_rowscale);
                for (int id : L.edown) add(id, resid_rowscale);
                add(L.sdown, resid_rowscale);
            }
        }
        const size_t bytes = static_cast<size_t>(off > 0 ? off : 1) * sizeof(float);
        if (off > 0 && folded.bytes < bytes) {
            if (folded.p) DLLM_TRY(check_hip(hipFree(folded.p), "hipFree"));
            folded.p = nullptr;
            DLLM_TRY(folded.alloc(bytes));
        }
        fold_on = off > 0;
        // the step's weight addresses changed: rebuild the transposes' job table and the qkv groups
        wt_jobs = nullptr;
        grp_rows = -1;
        ++tmpl_version;
        wt_valid = false;
        merged_valid = false;
        return kOk;
    }

    // rope_inv_freq with its scaling, and the attention factor (dllm_hip_trainer_set_rope).
    int set_rope(const double* host_inv_freq, int64_t pairs, double factor) {
        DLLM_REQUIRE(pairs == c.rotary_dim / 2, "set_rope needs rotary_dim / 2 inverse frequencies");
        DLLM_REQUIRE(factor > 0.0 && factor == factor, "the RoPE attention factor must be positive");
        DLLM_TRY(check_hip(hipDeviceSynchronize(), "set_rope"));
        DLLM_TRY(check_hip(hipMemcpy(inv_freq, host_inv_freq, static_cast<size_t>(pairs) * sizeof(double),
                                     hipMemcpyHostToDevice), "upload"));
        DLLM_TRY(launch_rope_tables(nullptr, T_max, inv_freq, c.rotary_dim / 2, cos_t, sin_t, nullptr));
        rope_factor = factor;
        if (factor != 1.0) {
            if (!rope_rowscale) DLLM_TRY(make(&rope_rowscale, static_cast<size_t>(QD)));
            std::vector<float> rs(static_cast<size_t>(QD));
            for (int64_t i = 0; i < QD; ++i) rs[static_cast<size_t>(i)] = (i % c.head_dim) < c.rotary_dim ? static_cast<float>(factor) : 1.0f;
            DLLM_TRY(check_hip(hipMemcpy(rope_rowscale, rs.data(), rs.size() * sizeof(float), hipMemcpyHostToDevice),
                               "upload"));
        }
        DLLM_TRY(setup_fold());
        return check_hip(hipDeviceSynchronize(), "set_rope");
    }
    float* G(int id) const { return grads.as<float>() + tensors[static_cast<size_t>(id)].offset; }
    float* WT(int id) const { return wt.as<float>() + tensors[static_cast<size_t>(id)].wt_offset; }
    const float* Popt(int id) const { return id >= 0 ? P(id) : nullptr; }

    // ---- weight gradients on a second stream ----
    // The backward's dense weight-gradient matmuls (and the bias column sums) read only buffers the input-gradient
    // chain has finished writing, plus the saved activations, and write only their own gradient tensors; each result
    // is the same launch on the same inputs whichever stream runs it. So they run on a second stream, overlapped with
    // the chain (whose small launches leave most CUs idle): a batch of them waits for the chain up to the point where
    // it is issued (the fork event), and the chain waits for a batch's completion event before it next overwrites a
    // buffer the batch reads. The stream is joined before the embedding gradients and the optimizer, which read every
    // gradient, and before the next step's forward rewrites the saved activations. While the matmuls are being timed
    // everything stays on the caller's stream, so each launch is timed alone.
    enum SideEvent { kSideDown, kSideMlp, kSideO, kSideQkv, kSideNormMlp, kSideNormAttn, kSideJoin, kSideEvents };
    hipStream_t side = nullptr;
    // a third stream for the attention backward's dq, which runs beside dk and dv (independent inputs and outputs)
    hipStream_t aux = nullptr;
    hipEvent_t aux_fork = nullptr, aux_done = nullptr;
    hipEvent_t side_fork = nullptr;
    hipEvent_t side_done[kSideEvents] = {};
    bool side_pending[kSideEvents] = {};
    bool side_on = false;  // this step's backward uses the second stream

    int side_setup() {
        if (side) return kOk;
        DLLM_TRY(check_hip(hipStreamCreateWithFlags(&side, hipStreamNonBlocking), "stream"));
        DLLM_TRY(check_hip(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking), "stream"));
        DLLM_TRY(check_hip(hipEventCreateWithFlags(&aux_fork, hipEventDisableTiming), "event"));
        DLLM_TRY(check_hip(hipEventCreateWithFlags(&aux_done, hipEventDisableTiming), "event"));
        DLLM_TRY(check_hip(hipEventCreateWithFlags(&side_fork, hipEventDisableTiming), "event"));
        for (hipEvent_t& e : side_done) DLLM_TRY(check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "event"));
        return kOk;
    }

    // The stream the next weight-gradient batch runs on, after it has been ordered behind the chain's work so far.
    int side_fork_from(hipStream_t s, hipStream_t* out) {
        if (!side_on) {
            *out = s;
            return kOk;
        }
        DLLM_TRY(check_hip(hipEventRecord(side_fork, s), "event"));
        DLLM_TRY(check_hip(hipStreamWaitEvent(side, side_fork, 0), "event"));
        *out = side;
        return kOk;
    }

    int side_mark(SideEvent e) {
        if (!side_on) return kOk;
        DLLM_TRY(check_hip(hipEventRecord(side_done[e], side), "event"));
        side_pending[e] = true;
        return kOk;
    }

    // The chain waits for the last batch marked `e` before overwriting what that batch reads.
    int side_wait(SideEvent e, hipStream_t s) {
        if (!side_on || !side_pending[e]) return kOk;
        side_pending[e] = false;
        return check_hip(hipStreamWaitEvent(s, side_done[e], 0), "event");
    }

    int side_join(hipStream_t s) {
        if (!side_on) return kOk;
        DLLM_TRY(check_hip(hipEventRecord(side_done[kSideJoin], side), "event"));
        DLLM_TRY(check_hip(hipStreamWaitEvent(s, side_done[kSideJoin], 0), "event"));
        for (bool& b : side_pending) b = false;
        side_on = false;
        return kOk;
    }

    // ---- matmul timing (dllm_hip_trainer_profile) ----
    bool profiling = false;
    std::vector<hipEvent_t> events;  // pairs
    size_t event_used = 0;
    double profile_flops = 0.0;
    int64_t profile_launches = 0;
    double profile_ms_done = 0.0;

    int drain_events() {
        for (size_t i = 0; i + 1 < event_used; i += 2) {
            DLLM_TRY(check_hip(hipEventSynchronize(events[i + 1]), "event"));
            float ms = 0.0f;
            DLLM_TRY(check_hip(hipEventElapsedTime(&ms, events[i], events[i + 1]), "event"));
            profile_ms_done += ms;
        }
        event_used = 0;
        return kOk;
    }

    int gemm(const GemmCall& g, hipStream_t s) {
        if (!profiling) return launch_gemm(g, s);
        DLLM_TRY(profile_begin(s));
        DLLM_TRY(launch_gemm(g, s));
        return profile_end(flops_of(g), s);
    }

    // One launch of a layer's expert matmuls (a group table made by group_rows).
    int gemm_group(const GemmGroup& grp, const void* table, double flops, hipStream_t s) {
        if (!profiling) return launch_gemm_group(grp, table, s);
        DLLM_TRY(profile_begin(s));
        DLLM_TRY(launch_gemm_group(grp, table, s));
        return profile_end(flops, s);
    }

    static double flops_of(const GemmCall& g) {
        const double L = static_cast<double>(g.l1 - g.l0);  // segmented calls set [l0, l1) to their whole row range
        return 2.0 * static_cast<double>(g.I) * static_cast<double>(g.J) * L;
    }

    int profile_begin(hipStream_t s) {
        if (event_used + 2 > events.size()) {
            if (events.size() >= 8192) DLLM_TRY(drain_events());
            while (event_used + 2 > events.size()) {
                hipEvent_t e;
                DLLM_TRY(check_hip(hipEventCreate(&e), "event"));
                events.push_back(e);
            }
        }
        return check_hip(hipEventRecord(events[event_used], s), "event");
    }

    int profile_end(double flops, hipStream_t s) {
        DLLM_TRY(check_hip(hipEventRecord(events[event_used + 1], s), "event"));
        event_used += 2;
        profile_flops += flops;
        profile_launches += 1;
        return kOk;
    }

    // W^T of every linear weight for the forward matmuls, in one launch (the job table is made on first use: the
    // weights' addresses, merged ones included, are fixed from then on).
    TransposeJob* wt_jobs = nullptr;
    int64_t* wt_tiles = nullptr;
    int wt_njobs = 0;
    int64_t wt_ntiles = 0;

    int refresh_transposes(hipStream_t s) {
        if (wt_jobs == nullptr) {
            std::vector<TransposeJob> jobs;
            for (size_t i = 0; i < tensors.size(); ++i) {
                const TensorInfo& t = tensors[i];
                if (t.wt_offset >= 0) jobs.push_back({P(static_cast<int>(i)), t.rows, t.cols, wt.as<float>() + t.wt_offset});
            }
            std::vector<int64_t> starts(jobs.size() + 1);
            wt_njobs = static_cast<int>(jobs.size());
            wt_ntiles = transpose_batch_tiles(jobs.data(), wt_njobs, starts.data());
            DLLM_TRY(make(&wt_jobs, std::max<size_t>(jobs.size(), 1)));
            DLLM_TRY(make(&wt_tiles, starts.size()));
            DLLM_TRY(check_hip(hipMemcpy(wt_jobs, jobs.data(), jobs.size() * sizeof(TransposeJob),
                                         hipMemcpyHostToDevice), "upload"));
            DLLM_TRY(check_hip(hipMemcpy(wt_tiles, starts.data(), starts.size() * 8, hipMemcpyHostToDevice), "upload"));
        }
        if (wt_njobs > 0) DLLM_TRY(launch_transpose_batch(wt_jobs, wt_tiles, wt_njobs, wt_ntiles, s));
        wt_valid = true;
        return kOk;
    }

    // The q, k and v projections of every layer read the same h1: one grouped launch per layer runs all three (their
    // tiles together fill the chip; k and v alone are 2 x 64 tiles at the c3 shapes). Each output's bits are those of
    // its own launch. The tables depend on the row count R and are rebuilt (after the stream drains) when it changes.
    // One grouped matmul launch per layer and kind (a table each, prepared per row count): the q/k/v forward and
    // the gate/up forward (independent outputs), and, when the row count is small enough that each of these
    // matmuls alone leaves CUs idle, the input gradients of gate/up and of q/k/v, each into its own buffer (dh,
    // dh_b, dh_c) and then added in the reference's order: dh2 = dx_gate + dx_up, dh1 = (dh_q + dh_k) + dh_v.
    enum LayerGroup { kGrpQkvFwd, kGrpMlpFwd, kGrpMlpDx, kGrpQkvDx, kLayerGroups };
    static constexpr int kGroupCap = 3;  // matmuls per group table
    char* grp_tables = nullptr;          // [layer][kind]
    std::vector<GemmGroup> grp;          // [layer * kLayerGroups + kind]
    bool grp_on[kLayerGroups] = {};
    std::vector<double> grp_flops;       // algorithmic flop of each group (matmul timing)
    int64_t grp_rows = -1;               // the row count the tables were prepared for
    float *dh_b = nullptr, *dh_c = nullptr;
    float* dh1 = nullptr;  // the attention block's input gradient (dh holds the MLP block's)

    const GemmGroup& group_of(int64_t l, int kind) const { return grp[static_cast<size_t>(l * kLayerGroups + kind)]; }
    const char* table_of(int64_t l, int kind) const {
        return grp_tables + gemm_group_bytes(kGroupCap) * static_cast<size_t>(l * kLayerGroups + kind);
    }

    int prepare_groups(int64_t R, hipStream_t s) {
        if (R == grp_rows) return kOk;
        const size_t gb = gemm_group_bytes(kGroupCap);
        const size_t n = static_cast<size_t>(c.layers) * kLayerGroups;
        if (grp_tables == nullptr) DLLM_TRY(make(&grp_tables, gb * n));
        std::vector<char> host(gb * n, 0);
        grp.assign(n, GemmGroup{});
        grp_flops.assign(n, 0.0);
        // the grouped kernel takes whole 16-byte chunks of the operands; other shapes keep one launch per matmul
        const bool rows_ok = R > 0 && H % 4 == 0;
        for (int k = 0; k < kLayerGroups; ++k) grp_on[k] = rows_ok && (E == 0 || k == kGrpQkvFwd || k == kGrpQkvDx);
        const float* dqf = c.qk_norm ? dq2 : dq;
        const float* dkf = c.qk_norm ? dk2 : dk;
        for (int64_t l = 0; l < c.layers; ++l) {
            const LayerIds& L = layer_ids[static_cast<size_t>(l)];
            Saved& sv = saved[static_cast<size_t>(l)];
            for (int k = 0; k < kLayerGroups; ++k) {
                if (!grp_on[k]) continue;
                GemmCall calls[kGroupCap];
                int nc = 0;
                if (k == kGrpQkvFwd) {
                    calls[nc++] = fwd_call(sv.h1, R, H, L.q, Popt(L.qb), sv.q_raw, nullptr);
                    calls[nc++] = fwd_call(sv.h1, R, H, L.k, Popt(L.kb), sv.k_raw, nullptr);
                    calls[nc++] = fwd_call(sv.h1, R, H, L.v, Popt(L.vb), sv.v, nullptr);
                } else if (k == kGrpMlpFwd) {
                    calls[nc++] = fwd_call(sv.h2, R, H, L.gate, nullptr, sv.gate, nullptr);
                    calls[nc++] = fwd_call(sv.h2, R, H, L.up, nullptr, sv.up, nullptr);
                } else if (k == kGrpMlpDx) {
                    calls[nc++] = dx_call(dgate, R, L.gate, dh, nullptr);
                    calls[nc++] = dx_call(dup, R, L.up, dh_b, nullptr);
                } else {
                    calls[nc++] = dx_call(dqf, R, L.q, dh1, nullptr);
                    calls[nc++] = dx_call(dkf, R, L.k, dh_b, nullptr);
                    calls[nc++] = dx_call(dv_t, R, L.v, dh_c, nullptr);
                }
                bool ok = true;
                for (int i = 0; i < nc; ++i)
                    ok = ok && gemm_mfma_shape(calls[i]) && calls[i].a_kind == calls[0].a_kind;
                GemmGroup& g = grp[static_cast<size_t>(l * kLayerGroups + k)];
                const size_t gi = static_cast<size_t>(l * kLayerGroups + k);
                if (ok) DLLM_TRY(gemm_group_prepare(calls, nc, kGroupCap, host.data() + gb * gi, &g));
                for (int i = 0; i < nc; ++i) grp_flops[gi] += flops_of(calls[i]);
                // the input-gradient groups only where the separate launches would take small tiles
                const bool dx_kind = k == kGrpMlpDx || k == kGrpQkvDx;
                if (!ok || (dx_kind && g.tile == 4)) grp_on[k] = false;
            }
        }
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "group tables"));  // no launch still reads the old tables
        DLLM_TRY(check_hip(hipMemcpy(grp_tables, host.data(), host.size(), hipMemcpyHostToDevice), "upload"));
        grp_rows = R;
        return kOk;
    }

    int group_launch(int64_t l, int kind, hipStream_t s) {
        const size_t i = static_cast<size_t>(l * kLayerGroups + kind);
        return gemm_group(grp[i], table_of(l, kind), grp_flops[i], s);
    }

    int qkv_forward(int64_t l, int64_t R, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        Saved& sv = saved[static_cast<size_t>(l)];
        if (grp_on[kGrpQkvFwd] && grp_rows == R) return group_launch(l, kGrpQkvFwd, s);
        DLLM_TRY(linear_fwd(sv.h1, R, H, L.q, Popt(L.qb), sv.q_raw, nullptr, s));
        DLLM_TRY(linear_fwd(sv.h1, R, H, L.k, Popt(L.kb), sv.k_raw, nullptr, s));
        return linear_fwd(sv.h1, R, H, L.v, Popt(L.vb), sv.v, nullptr, s);
    }

    // out[R][N] (+)= x[R][K] @ W^T (+ bias); the matmul reads x itself (A transposed: A[k][r] = x[r][k]).
    int linear_fwd(const float* x, int64_t R, int64_t K, int w_id, const float* bias, float* out, const float* addsrc,
                   hipStream_t s) {
        return gemm(fwd_call(x, R, K, w_id, bias, out, addsrc), s);
    }

    GemmCall fwd_call(const float* x, int64_t R, int64_t K, int w_id, const float* bias, float* out,
                      const float* addsrc) const {
        const int64_t N = tensors[static_cast<size_t>(w_id)].rows;
        GemmCall g;
        g.Af = x;
        g.a_kind = 2;
        g.lda = K;
        g.B = WT(w_id);
        g.ldb = N;
        g.C = out;
        g.ldc = N;
        g.I = R;
        g.J = N;
        g.l0 = 0;
        g.l1 = K;
        g.bias = bias;
        g.addsrc = addsrc;
        g.ld_add = N;
        g.a_scratch = mm_scratch;
        g.a_scratch_cap = mm_scratch_cap;
        return g;
    }

    // dx[R][K] (= addsrc +) sum_n dy[r][n] W[n][k]; the matmul reads dy[R][N] itself (A transposed).
    int linear_dx(const float* dyv, int64_t R, int w_id, float* out, const float* addsrc, hipStream_t s) {
        return gemm(dx_call(dyv, R, w_id, out, addsrc), s);
    }

    GemmCall dx_call(const float* dyv, int64_t R, int w_id, float* out, const float* addsrc) const {
        const TensorInfo& t = tensors[static_cast<size_t>(w_id)];
        GemmCall g;
        g.Af = dyv;
        g.a_kind = 2;
        g.lda = t.rows;
        g.B = P(w_id);
        g.ldb = t.cols;
        g.C = out;
        g.ldc = t.cols;
        g.I = R;
        g.J = t.cols;
        g.l0 = 0;
        g.l1 = t.rows;
        g.addsrc = addsrc;
        g.ld_add = t.cols;
        g.a_scratch = mm_scratch;
        g.a_scratch_cap = mm_scratch_cap;
        return g;
    }

    // grad[w] = window-ordered float sum of per-window dW = sum over window rows of dy[r][n] x[r][k]. The windows are
    // the step's (seg_d), or those of an expert's group (seg, over `rows` grouped rows).
    int linear_dw(const float* dyv, int64_t N, const float* x, int64_t K, int nseg, float* out, const int* addrow_,
                  const float* addend, hipStream_t s, const int64_t* seg = nullptr, int64_t rows = -1,
                  const float* rowscale = nullptr) {
        if (!grad_wanted(out)) return kOk;
        GemmCall g = dw_call(dyv, N, x, K, nseg, out, addrow_, addend, seg, rows);
        g.seg_rowscale = rowscale;
        return gemm(g, s);
    }

    GemmCall dw_call(const float* dyv, int64_t N, const float* x, int64_t K, int nseg, float* out, const int* addrow_,
                     const float* addend, const int64_t* seg = nullptr, int64_t rows = -1) const {
        GemmCall g;
        g.Af = dyv;  // A rows: A[r][n] = dy[r][n]
        g.a_kind = 1;
        g.lda = N;
        g.B = x;
        g.ldb = K;
        g.C = out;
        g.ldc = K;
        g.I = N;
        g.J = K;
        g.seg = seg ? seg : seg_d;
        g.nseg = nseg;
        g.l0 = 0;
        g.l1 = seg ? rows : seg_host.back();
        g.seg_addrow = addrow_;
        g.seg_addend = addend;
        g.ld_seg_add = K;
        g.seg_partial = gemm_part;
        g.seg_partial_cap = gemm_part_cap;
        g.seg_weight = window_weights();
        g.a_scratch = mm_scratch;
        g.a_scratch_cap = mm_scratch_cap;
        return g;
    }

    int norm_dw(const float* dyv, const float* x, const double* inv, int64_t dim, int64_t rows_per_token, int nseg,
                float* out, hipStream_t s, const float* colscale = nullptr) {
        if (!grad_wanted(out)) return kOk;
        std::vector<int64_t> seg(seg_host.size());
        for (size_t i = 0; i < seg.size(); ++i) seg[i] = seg_host[i] * rows_per_token;
        return launch_column_sums(1, dyv, x, inv, dim, seg.data(), nseg, s == side && side_on ? col_part_side : col_part,
                                  out, s, window_weights(), colscale);
    }

    // ---- attention (attn_lds.hip, attn_chains.hip) ----
    int64_t nwin = 0;  // windows of the current step

    double* et_of(int64_t l) const { return attn_et + l * W_max * c.heads * Tp * Tp; }
    double* inv_of(int64_t l) const { return attn_inv + l * W_max * c.heads * Tp; }
    double* slope_of(int64_t l) const { return attn_slope + l * W_max * c.heads * Tp * Tp; }

    // attention() of every (window, head) of the step (nn.hpp:761-796): S^T = K Q^T scale, the softmax chains per
    // query, out = (E V) inv.
    int attention_forward(int64_t l, const Saved& sv, const AttentionBatch& b, hipStream_t s) {
        const int64_t nh = c.heads, nkv = c.kv_heads, hd = c.head_dim, G = nh / nkv, n = b.max_q;
        DLLM_TRY(launch_heads_transpose(sv.q, QD, hd, attn_qt, false, Tp, hd * Tp, seg_d, nwin, nh, n, s));
        double* et = et_of(l);
        AttnTileCall g;
        g.seg = seg_d;
        g.windows = nwin;
        g.heads = nh;
        g.max_len = n;
        g.head_dim = hd;
        g.group = G;
        g.window = layer_window(l);
        // S^T[j][t] = sum_i k[j][i] q[t][i], times scale: A = the key rows themselves, read transposed
        g.A = AttnOperand{sv.k, 0, KVD, hd, G, KVD, 0, 1};
        g.a_float = true;
        g.a_row_alloc = hd;
        g.B = AttnOperand{attn_qt, nh * hd * Tp, 0, hd * Tp, 1, Tp, 0, 1};
        g.C = AttnOperand{et, nh * Tp * Tp, 0, Tp * Tp, 1, Tp, 0, 1};
        g.rows_kind = 0;
        g.cols_kind = 0;
        g.L = hd;
        g.mask = kMaskTileCausal;
        g.cols_per_lane = 4;
        g.b_row_alloc = Tp;
        g.exact_products = true;
        g.out_double = true;
        g.out_scale = c.attention_scale;
        const bool capped = c.attention_softcap != 0.0;  // the tiles' maxima are of the uncapped scores
        g.tile_max = capped ? nullptr : attn_tmax;
        g.tile_max_zstride = (Tp / 64) * Tp;
        g.tile_max_ld = Tp;
        DLLM_TRY(launch_attn_tiles(g, s));
        if (capped) DLLM_TRY(launch_softcap_scores(et, slope_of(l), nwin * nh * Tp * Tp, c.attention_softcap, s));
        DLLM_TRY(launch_softmax_rows(et, Tp, Tp * Tp, seg_d, nwin, nh, n, layer_window(l), inv_of(l), Tp, s,
                                     g.tile_max, (Tp / 64) * Tp, Tp));
        // out[t] = f32((sum_j e_j v_j) inv_t)
        AttnTileCall o = g;
        o.tile_max = nullptr;
        o.A = AttnOperand{et, nh * Tp * Tp, 0, Tp * Tp, 1, Tp, 0, 1};
        o.a_float = false;
        o.B = AttnOperand{sv.v, 0, KVD, hd, G, KVD, 0, 1};
        o.C = AttnOperand{sv.attended, 0, QD, hd, 1, QD, 0, 1};
        o.rows_kind = 0;
        o.cols_kind = 1;
        o.L = 0;
        o.mask = kMaskQueryRows;
        o.cols_per_lane = value_cols(n, nh, 1);
        o.b_row_alloc = 0;
        o.exact_products = false;
        o.out_double = false;
        o.rowscale = inv_of(l);
        o.rowscale_zstride = Tp;
        return launch_attn_tiles(o, s);
    }

    // Columns per lane of a head_dim-wide attention output launch (attn_value_cols).
    int value_cols(int64_t rows, int64_t heads, int64_t sets) const {
        return attn_value_cols(rows, c.head_dim, heads, nwin, sets);
    }

    // attention_backward (grad.hpp:206-301) of every (window, head): dq_t, dk_t, dv_t from dattended.
    int attention_backward(int64_t l, const Saved& sv, const AttentionBatch& b, hipStream_t s) {
        const int64_t nh = c.heads, nkv = c.kv_heads, hd = c.head_dim, G = nh / nkv, n = b.max_q;
        double* et = et_of(l);
        DLLM_TRY(launch_heads_transpose(dattended, QD, hd, attn_dot, false, Tp, hd * Tp, seg_d, nwin, nh, n, s));
        AttnTileCall g;
        g.seg = seg_d;
        g.windows = nwin;
        g.heads = nh;
        g.max_len = n;
        g.head_dim = hd;
        g.group = G;
        g.window = layer_window(l);
        // dP^T[j][t] = sum_i v[j][i] dout[t][i]
        g.A = AttnOperand{sv.v, 0, KVD, hd, G, KVD, 0, 1};
        g.a_float = true;
        g.a_row_alloc = hd;
        g.B = AttnOperand{attn_dot, nh * hd * Tp, 0, hd * Tp, 1, Tp, 0, 1};
        g.C = AttnOperand{attn_dpt, nh * Tp * Tp, 0, Tp * Tp, 1, Tp, 0, 1};
        g.rows_kind = 0;
        g.cols_kind = 0;
        g.L = hd;
        g.mask = kMaskTileCausal;
        g.cols_per_lane = 4;
        g.b_row_alloc = Tp;
        g.exact_products = true;
        g.out_double = true;
        g.out_scale = 1.0;
        DLLM_TRY(launch_attn_tiles(g, s));
        // D, p = e inv and ds = p (dp - D) scale: ds over dP^T (dq's operand), p and ds in the key-row layout
        // [w][g][(t, hh)][j] of dk and dv
        const int64_t gz = Tp * G * Tp;
        DLLM_TRY(launch_dsoftmax_regroup(et, attn_dpt, Tp, Tp * Tp, seg_d, nwin, nh, G, n, layer_window(l), inv_of(l),
                                         Tp, c.attention_scale, attn_dvec, attn_pg, attn_dsg, Tp, gz, s,
                                         c.attention_softcap != 0.0 ? slope_of(l) : nullptr));
        // dq[t] = sum_j ds[t][j] k[j]
        AttnTileCall q = g;
        q.A = AttnOperand{attn_dpt, nh * Tp * Tp, 0, Tp * Tp, 1, Tp, 0, 1};
        q.a_float = false;
        q.B = AttnOperand{sv.k, 0, KVD, hd, G, KVD, 0, 1};
        q.C = AttnOperand{dq_t, 0, QD, hd, 1, QD, 0, 1};
        q.cols_kind = 1;
        q.L = 0;
        q.mask = kMaskQueryRows;
        q.cols_per_lane = value_cols(n, nh, 1);
        q.b_row_alloc = 0;
        q.exact_products = false;
        q.out_double = false;
        hipStream_t qs = s;  // dq beside dk and dv: it reads the dS rows and k, they read p, ds, q and dout
        if (side_on) {
            DLLM_TRY(check_hip(hipEventRecord(aux_fork, s), "event"));
            DLLM_TRY(check_hip(hipStreamWaitEvent(aux, aux_fork, 0), "event"));
            qs = aux;
        }
        DLLM_TRY(launch_attn_tiles(q, qs));
        // dk[j] = sum over (t, hh) of ds q and dv[j] = sum of p dout, in one launch
        AttnTileCall k = q;
        k.heads = nkv;
        k.A = AttnOperand{attn_dsg, nkv * gz, 0, gz, 1, Tp, 0, 1};
        k.B = AttnOperand{sv.q, 0, QD, G * hd, 1, QD, hd, G};
        k.C = AttnOperand{dk_t, 0, KVD, hd, 1, KVD, 0, 1};
        k.second = true;
        k.A2 = AttnOperand{attn_pg, nkv * gz, 0, gz, 1, Tp, 0, 1};
        k.B2 = AttnOperand{dattended, 0, QD, G * hd, 1, QD, hd, G};
        k.C2 = AttnOperand{dv_t, 0, KVD, hd, 1, KVD, 0, 1};
        k.mask = kMaskKeyRows;
        k.cols_per_lane = value_cols(n, nkv, 2);
        DLLM_TRY(launch_attn_tiles(k, s));
        if (qs != s) {  // everything after reads dq_t, and the next layer rewrites the dS rows
            DLLM_TRY(check_hip(hipEventRecord(aux_done, qs), "event"));
            DLLM_TRY(check_hip(hipStreamWaitEvent(s, aux_done, 0), "event"));
        }
        return kOk;
    }

    // One layer's forward (backprop.py:423-487).
    int forward_layer(int64_t l, int64_t R, const AttentionBatch& b, float* x_out, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        Saved& sv = saved[static_cast<size_t>(l)];
        const double eps = c.rms_norm_eps;
        if (pre_norms()) DLLM_TRY(launch_rms_norm(sv.x_in, P(L.attn_norm), sv.h1, R, H, eps, uo(), nullptr, s));
        DLLM_TRY(qkv_forward(l, R, s));
        const float* qsrc = sv.q_raw;
        const float* ksrc = sv.k_raw;
        if (c.qk_norm == 2) {
            DLLM_TRY(launch_rms_norm(sv.q_raw, P(L.qn), sv.qn, R, QD, eps, uo(), nullptr, s));
            DLLM_TRY(launch_rms_norm(sv.k_raw, P(L.kn), sv.kn, R, KVD, eps, uo(), nullptr, s));
            qsrc = sv.qn;
            ksrc = sv.kn;
        } else if (c.qk_norm == 1) {
            DLLM_TRY(launch_rms_norm(sv.q_raw, P(L.qn), sv.qn, R * c.heads, c.head_dim, eps, uo(), nullptr, s));
            DLLM_TRY(launch_rms_norm(sv.k_raw, P(L.kn), sv.kn, R * c.kv_heads, c.head_dim, eps, uo(), nullptr, s));
            qsrc = sv.qn;
            ksrc = sv.kn;
        }
        DLLM_TRY(launch_rope_pair(qsrc, sv.q, c.heads, ksrc, sv.k, c.kv_heads, pos_index, cos_of(l), sin_of(l), R, c.head_dim,
                                  c.rotary_dim, 0, s));
        DLLM_TRY(attention_forward(l, sv, b, s));
        if (post_norms()) {  // x_mid = x + post_norm(out)
            DLLM_TRY(linear_fwd(sv.attended, R, QD, L.o, nullptr, sv.out, nullptr, s));
            DLLM_TRY(launch_rms_norm(sv.out, P(L.attn_post), post_tmp, R, H, eps, uo(), nullptr, s));
            DLLM_TRY(launch_add(sv.x_in, post_tmp, sv.x_mid, R * H, s));
        } else {
            DLLM_TRY(linear_fwd(sv.attended, R, QD, L.o, nullptr, sv.x_mid, sv.x_in, s));  // x_mid = x + out
        }
        if (pre_norms()) DLLM_TRY(launch_rms_norm(sv.x_mid, P(L.mlp_norm), sv.h2, R, H, eps, uo(), nullptr, s));
        if (sparse(l)) return moe_forward(l, R, x_out, s);
        if (grp_on[kGrpMlpFwd] && grp_rows == R) {
            DLLM_TRY(group_launch(l, kGrpMlpFwd, s));
        } else {
            DLLM_TRY(linear_fwd(sv.h2, R, H, L.gate, nullptr, sv.gate, nullptr, s));
            DLLM_TRY(linear_fwd(sv.h2, R, H, L.up, nullptr, sv.up, nullptr, s));
        }
        DLLM_TRY(launch_swiglu_forward(sv.gate, sv.up, sv.gate_act, sv.product, R * I, s, act()));
        if (post_norms()) {  // x_out = x_mid + post_norm(mlp)
            DLLM_TRY(linear_fwd(sv.product, R, I, L.down, nullptr, sv.mlp, nullptr, s));
            return mlp_post_norm(l, R, x_out, s);
        }
        return linear_fwd(sv.product, R, I, L.down, nullptr, x_out, sv.x_mid, s);  // x_out = x_mid + mlp
    }

    // One layer's backward (backprop.py:208-306); dx holds the gradient of the layer output on entry and of its input
    // on exit.
    int backward_layer(int64_t l, int64_t R, int nseg, const AttentionBatch& b, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        const Saved& sv = saved[static_cast<size_t>(l)];
        const double eps = c.rms_norm_eps;
        hipStream_t ws = s;  // the stream of the weight-gradient batches
        // post norms (backprop.py:224-229): the MLP's output gradient through its norm (one stream: side is off)
        const float* dmlp = dx;
        if (post_norms()) {
            DLLM_TRY(launch_rms_norm_backward_dx(sv.mlp, P(L.mlp_post), dx, dpost, nullptr, R, H, eps, uo(), inv_post, s));
            DLLM_TRY(norm_dw(dx, sv.mlp, inv_post, H, 1, nseg, G(L.mlp_post), s));
            dmlp = dpost;
        }
        if (sparse(l)) {
            DLLM_TRY(side_wait(kSideMlp, s));      // the previous layer's router dW reads dlogits_r
            DLLM_TRY(side_wait(kSideNormMlp, s));  // its mlp norm's dW reads dh
            DLLM_TRY(moe_backward(l, R, nseg, dmlp, s));
        } else {
            // SwiGLU (backprop.py:289-306)
            DLLM_TRY(linear_dx(dmlp, R, L.down, dproduct, nullptr, s));
            DLLM_TRY(side_fork_from(s, &ws));
            DLLM_TRY(linear_dw(dmlp, H, sv.product, I, nseg, G(L.down), nullptr, nullptr, ws, nullptr, -1,
                               unfold_scale(L.down)));
            DLLM_TRY(side_mark(kSideDown));
            DLLM_TRY(side_wait(kSideMlp, s));  // the previous layer's gate and up dW read dgate, dup
            DLLM_TRY(launch_swiglu_backward(sv.gate, sv.up, sv.gate_act, dproduct, dgate, dup, R * I, s, act()));
            DLLM_TRY(side_fork_from(s, &ws));
            DLLM_TRY(linear_dw(dgate, I, sv.h2, H, nseg, G(L.gate), nullptr, nullptr, ws));
            DLLM_TRY(linear_dw(dup, I, sv.h2, H, nseg, G(L.up), nullptr, nullptr, ws));
            DLLM_TRY(side_mark(kSideMlp));
            DLLM_TRY(side_wait(kSideNormMlp, s));  // the previous layer's mlp norm dW reads dh
            if (grp_on[kGrpMlpDx] && grp_rows == R) {
                DLLM_TRY(group_launch(l, kGrpMlpDx, s));
                DLLM_TRY(launch_add(dh, dh_b, dh, R * H, s));  // dh2 = dx_gate + dx_up
            } else {
                DLLM_TRY(linear_dx(dgate, R, L.gate, dh, nullptr, s));
                DLLM_TRY(linear_dx(dup, R, L.up, dh, dh, s));  // dh2 = dx_gate + dx_up
            }
        }
        // mlp norm; dx_mid = dx + dh2'
        DLLM_TRY(side_wait(kSideO, s));  // the previous layer's o dW reads dx_mid
        if (pre_norms()) {
            DLLM_TRY(launch_rms_norm_backward_dx(sv.x_mid, P(L.mlp_norm), dh, dx_mid, dx, R, H, eps, uo(), inv_mlp, s));
            DLLM_TRY(side_fork_from(s, &ws));
            DLLM_TRY(norm_dw(dh, sv.x_mid, inv_mlp, H, 1, nseg, G(L.mlp_norm), ws));
            DLLM_TRY(side_mark(kSideNormMlp));
        } else {
            DLLM_TRY(launch_add(dx, dh, dx_mid, R * H, s));  // dx_mid = dx + dh2
        }
        // attention output projection (through its post norm, backprop.py:237-242)
        const float* dout = dx_mid;
        if (post_norms()) {
            DLLM_TRY(launch_rms_norm_backward_dx(sv.out, P(L.attn_post), dx_mid, dpost, nullptr, R, H, eps, uo(), inv_post,
                                                 s));
            DLLM_TRY(norm_dw(dx_mid, sv.out, inv_post, H, 1, nseg, G(L.attn_post), s));
            dout = dpost;
        }
        DLLM_TRY(linear_dx(dout, R, L.o, dattended, nullptr, s));
        DLLM_TRY(side_fork_from(s, &ws));
        DLLM_TRY(linear_dw(dout, H, sv.attended, QD, nseg, G(L.o), nullptr, nullptr, ws, nullptr, -1,
                           unfold_scale(L.o)));
        DLLM_TRY(side_mark(kSideO));
        DLLM_TRY(side_wait(kSideQkv, s));  // the previous layer's q/k/v dW read dq, dk (dq2, dk2) and dv_t
        DLLM_TRY(attention_backward(l, sv, b, s));
        DLLM_TRY(launch_rope_pair(dq_t, dq, c.heads, dk_t, dk, c.kv_heads, pos_index, cos_of(l), sin_of(l), R, c.head_dim,
                                  c.rotary_dim, 1, s));
        const float* dqf = dq;
        const float* dkf = dk;
        if (c.qk_norm == 1) {
            DLLM_TRY(launch_rms_norm_backward_dx(sv.q_raw, P(L.qn), dq, dq2, nullptr, R * c.heads, c.head_dim, eps, uo(),
                                                 inv_rms, s));
            DLLM_TRY(norm_dw(dq, sv.q_raw, inv_rms, c.head_dim, c.heads, nseg, G(L.qn), s, unfold_scale(L.qn)));
            DLLM_TRY(launch_rms_norm_backward_dx(sv.k_raw, P(L.kn), dk, dk2, nullptr, R * c.kv_heads, c.head_dim, eps,
                                                 uo(), inv_rms, s));
            DLLM_TRY(norm_dw(dk, sv.k_raw, inv_rms, c.head_dim, c.kv_heads, nseg, G(L.kn), s, unfold_scale(L.kn)));
            dqf = dq2;
            dkf = dk2;
        } else if (c.qk_norm == 2) {
            DLLM_TRY(launch_rms_norm_backward_dx(sv.q_raw, P(L.qn), dq, dq2, nullptr, R, QD, eps, uo(), inv_rms, s));
            DLLM_TRY(norm_dw(dq, sv.q_raw, inv_rms, QD, 1, nseg, G(L.qn), s, unfold_scale(L.qn)));
            DLLM_TRY(launch_rms_norm_backward_dx(sv.k_raw, P(L.kn), dk, dk2, nullptr, R, KVD, eps, uo(), inv_rms, s));
            DLLM_TRY(norm_dw(dk, sv.k_raw, inv_rms, KVD, 1, nseg, G(L.kn), s, unfold_scale(L.kn)));
            dqf = dq2;
            dkf = dk2;
        }
        // q, k, v projections: dh1 = (dh_q + dh_k) + dh_v
        const float* ds[3] = {dqf, dkf, dv_t};
        const int ws_[3] = {L.q, L.k, L.v};
        const int bs_[3] = {L.qb, L.kb, L.vb};
        const int64_t ns[3] = {QD, KVD, KVD};
        DLLM_TRY(side_fork_from(s, &ws));
        for (int p = 0; p < 3; ++p) {
            DLLM_TRY(linear_dw(ds[p], ns[p], sv.h1, H, nseg, G(ws_[p]), nullptr, nullptr, ws, nullptr, -1,
                               unfold_scale(ws_[p])));
            if (bs_[p] >= 0 && grad_wanted(G(bs_[p])))
                DLLM_TRY(launch_column_sums(0, ds[p], nullptr, nullptr, ns[p], seg_host.data(), nseg,
                                            ws == s ? col_part : col_part_side, G(bs_[p]), ws, window_weights(),
                                            unfold_scale(bs_[p])));
        }
        DLLM_TRY(side_mark(kSideQkv));
        DLLM_TRY(side_wait(kSideNormAttn, s));  // the previous layer's attention norm dW reads dh1
        if (grp_on[kGrpQkvDx] && grp_rows == R) {
            DLLM_TRY(group_launch(l, kGrpQkvDx, s));
            DLLM_TRY(launch_add3(dh1, dh_b, dh_c, dh1, R * H, s));  // (dh_q + dh_k) + dh_v
        } else {
            for (int p = 0; p < 3; ++p) DLLM_TRY(linear_dx(ds[p], R, ws_[p], dh1, p == 0 ? nullptr : dh1, s));
        }
        // attention norm; dx = dx_mid + dh1'
        DLLM_TRY(side_wait(kSideDown, s));  // this layer's down dW reads dx
        if (!pre_norms()) return launch_add(dx_mid, dh1, dx, R * H, s);
        DLLM_TRY(launch_rms_norm_backward_dx(sv.x_in, P(L.attn_norm), dh1, dx, dx_mid, R, H, eps, uo(), inv_attn, s));
        DLLM_TRY(side_fork_from(s, &ws));
        DLLM_TRY(norm_dw(dh1, sv.x_in, inv_attn, H, 1, nseg, G(L.attn_norm), ws));
        return side_mark(kSideNormAttn);
    }

    // ---- routed experts (backprop.py:308-377, 501-527) ----

    // Groups the step's rows by expert from the layer's choices (host; the choices come back first): experts
    // ascending, within an expert rows ascending (np.nonzero), and the per-window split of each group.
    int group_rows_host(int64_t l, Saved& sv, int64_t R, hipStream_t s) {
        std::vector<int64_t> chosen(static_cast<size_t>(R * K));
        DLLM_TRY(check_hip(hipMemcpyAsync(chosen.data(), sv.chosen, chosen.size() * 8, hipMemcpyDeviceToHost, s),
                           "download"));
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "routing"));
        const int64_t nw = nwin;
        std::vector<int64_t> count(static_cast<size_t>(E), 0);
        for (int64_t i = 0; i < R * K; ++i) {
            const int64_t e = chosen[static_cast<size_t>(i)];
            DLLM_REQUIRE(e >= 0 && e < E, "routing produced an expert out of range");
            ++count[static_cast<size_t>(e)];
        }
        sv.estart.assign(static_cast<size_t>(E + 1), 0);
        for (int64_t e = 0; e < E; ++e) sv.estart[static_cast<size_t>(e + 1)] = sv.estart[e] + count[e];
        std::vector<int64_t> fill(sv.estart.begin(), sv.estart.end() - 1);
        std::vector<int64_t> row_of(static_cast<size_t>(R * K)), slot(row_of.size()), order(row_of.size());
        std::vector<int64_t> eseg(static_cast<size_t>(E * (W_max + 1)), 0);
        std::vector<std::pair<int64_t, int64_t>> pick(static_cast<size_t>(K));
        int64_t w = 0;
        for (int64_t r = 0; r < R; ++r) {
            while (seg_host[static_cast<size_t>(w + 1)] <= r) ++w;
            for (int64_t j = 0; j < K; ++j) {
                const int64_t e = chosen[static_cast<size_t>(r * K + j)];
                const int64_t p = fill[static_cast<size_t>(e)]++;
                row_of[static_cast<size_t>(p)] = r;
                slot[static_cast<size_t>(p)] = r * K + j;
                ++eseg[static_cast<size_t>(e * (W_max + 1) + w + 1)];
                ++counts_host[static_cast<size_t>(w * E + e)];
            }
            // the row's positions by ascending expert (a row chooses an expert at most once)
            for (int64_t j = 0; j < K; ++j) {
                const int64_t e = chosen[static_cast<size_t>(r * K + j)];
                pick[static_cast<size_t>(j)] = {e, fill[static_cast<size_t>(e)] - 1};
            }
            std::sort(pick.begin(), pick.end());
            for (int64_t j = 0; j < K; ++j) order[static_cast<size_t>(r * K + j)] = pick[static_cast<size_t>(j)].second;
        }
        for (int64_t e = 0; e < E; ++e)
            for (int64_t i = 1; i <= nw; ++i) eseg[static_cast<size_t>(e * (W_max + 1) + i)] +=
                eseg[static_cast<size_t>(e * (W_max + 1) + i - 1)];
        DLLM_TRY(check_hip(hipMemcpyAsync(sv.row_of, row_of.data(), row_of.size() * 8, hipMemcpyHostToDevice, s),
                           "upload"));
        DLLM_TRY(check_hip(hipMemcpyAsync(sv.slot, slot.data(), slot.size() * 8, hipMemcpyHostToDevice, s), "upload"));
        DLLM_TRY(check_hip(hipMemcpyAsync(sv.order, order.data(), order.size() * 8, hipMemcpyHostToDevice, s),
                           "upload"));
        DLLM_TRY(check_hip(hipMemcpyAsync(sv.eseg, eseg.data(), eseg.size() * 8, hipMemcpyHostToDevice, s), "upload"));
        std::vector<char> tables;
        DLLM_TRY(expert_tables(l, sv, &tables));
        DLLM_TRY(check_hip(hipMemcpyAsync(sv.tables, tables.data(), tables.size(), hipMemcpyHostToDevice, s),
                           "upload"));
        // the host vectors die here: wait for the copies
        return check_hip(hipStreamSynchronize(s), "grouping");
    }

    // The layer's nine kinds of expert matmuls over the grouped rows (expert e's rows are st .. st + n - 1):
    //   forward  gate/up = xg W^T, y = product Wd^T;  backward  dproduct = dy Wd, dxg = dgate Wg (+ dup Wu),
    //   and each weight's dW over the expert's rows split at the window boundaries.
    // Expert e's matmul of one kind over its grouped rows st .. st + n - 1; false when the gradient it forms reaches
    // no optimizer (LoRA runs without that target).
    bool expert_call(const LayerIds& L, const Saved& sv, int kind, int64_t e, int64_t st, int64_t n, GemmCall* out) const {
        const int64_t* es = sv.eseg + e * (W_max + 1);
        GemmCall g;
        switch (kind) {
            case kFwdGate: g = fwd_call(xg + st * H, n, H, L.egate[e], nullptr, sv.gate + st * EI, nullptr); break;
            case kFwdUp: g = fwd_call(xg + st * H, n, H, L.eup[e], nullptr, sv.up + st * EI, nullptr); break;
            case kFwdDown: g = fwd_call(sv.product + st * EI, n, EI, L.edown[e], nullptr, sv.y + st * H, nullptr); break;
            case kDxDown: g = dx_call(dyg + st * H, n, L.edown[e], dproduct + st * EI, nullptr); break;
            case kDwDown:
                if (!grad_wanted(G(L.edown[e]))) return false;
                g = dw_call(dyg + st * H, H, sv.product + st * EI, EI, static_cast<int>(nwin), G(L.edown[e]), nullptr,
                            nullptr, es, n);
                g.seg_rowscale = unfold_scale(L.edown[e]);
                break;
            case kDxGate: g = dx_call(dgate + st * EI, n, L.egate[e], dxg + st * H, nullptr); break;
            case kDwGate:
                if (!grad_wanted(G(L.egate[e]))) return false;
                g = dw_call(dgate + st * EI, EI, xg + st * H, H, static_cast<int>(nwin), G(L.egate[e]), nullptr,
                            nullptr, es, n);
                break;
            case kDxUp: g = dx_call(dup + st * EI, n, L.eup[e], dxg + st * H, dxg + st * H); break;
            default:
                if (!grad_wanted(G(L.eup[e]))) return false;
                g = dw_call(dup + st * EI, EI, xg + st * H, H, static_cast<int>(nwin), G(L.eup[e]), nullptr, nullptr, es,
                            n);
                break;
        }
        g.seg_partial = nullptr;
        g.seg_partial_cap = 0;
        *out = g;
        return true;
    }

    // How each kind's operands advance per grouped row (the fill kernel's shifts of the template table).
    GemmRowShift expert_shift(int kind) const {
        GemmRowShift sh;
        switch (kind) {
            case kFwdGate: case kFwdUp: sh.a = H; sh.c = EI; break;
            case kFwdDown: sh.a = EI; sh.c = H; break;
            case kDxDown: sh.a = H; sh.c = EI; break;
            case kDxGate: sh.a = EI; sh.c = H; break;
            case kDxUp: sh.a = EI; sh.c = H; sh.add = H; break;
            case kDwDown: sh.a = H; sh.b = EI; sh.rows_in_reduction = 1; break;
            default: sh.a = EI; sh.b = H; sh.rows_in_reduction = 1; break;  // kDwGate, kDwUp
        }
        return sh;
    }

    // The layer's nine kinds of expert matmuls over the grouped rows (expert e's rows are st .. st + n - 1):
    //   forward  gate/up = xg W^T, y = product Wd^T;  backward  dproduct = dy Wd, dxg = dgate Wg (+ dup Wu),
    //   and each weight's dW over the expert's rows split at the window boundaries. Host grouping (model sizes the
    //   grouped kernel cannot stage): the tables from the host's group starts.
    int expert_tables(int64_t l, Saved& sv, std::vector<char>* out) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        const size_t gb = gemm_group_bytes(static_cast<int>(E));
        out->assign(kExpertMatmuls * gb, 0);
        std::vector<GemmCall> calls;
        for (int kind = 0; kind < kExpertMatmuls; ++kind) {
            calls.clear();
            for (int64_t e = 0; e < E; ++e) {
                GemmCall g;
                if (expert_call(L, sv, kind, e, sv.estart[e], sv.estart[e + 1] - sv.estart[e], &g)) calls.push_back(g);
            }
            GemmGroup& grp = sv.groups[kind];
            grp = GemmGroup{};
            sv.group_flops[kind] = 0.0;
            sv.loose[kind].clear();
            if (calls.empty()) continue;
            bool grouped = true;
            for (const GemmCall& g : calls) grouped = grouped && gemm_mfma_shape(g);
            if (!grouped) {
                sv.loose[kind] = calls;
                continue;
            }
            DLLM_TRY(gemm_group_prepare(calls.data(), static_cast<int>(calls.size()), static_cast<int>(E),
                                        out->data() + kind * gb, &grp));
            for (const GemmCall& g : calls) sv.group_flops[kind] += flops_of(g);
        }
        return kOk;
    }

    // Device grouping: each kind's template table (every expert at grouped row 0 with no rows), rebuilt only when the
    // step's shape (rows, windows, DPO factors) or the weights' addresses change. The plain kinds take the tile size
    // an even spread of the rows over the experts would take (as gemm_group_prepare); the bits do not depend on it.
    int expert_templates(int64_t l, Saved& sv, int64_t R, hipStream_t s) {
        const std::vector<int64_t> key = {R, nwin, dpo.on ? 1 : 0, tmpl_version};
        if (sv.tmpl_key == key) return kOk;
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        const size_t gb = gemm_group_bytes(static_cast<int>(E));
        std::vector<char> host(kExpertMatmuls * gb, 0);
        std::vector<GemmCall> calls(static_cast<size_t>(E));
        const int64_t even = ceil_div(R * K, E);  // rows per expert if the choices spread evenly
        for (int kind = 0; kind < kExpertMatmuls; ++kind) {
            GemmGroup& grp = sv.groups[kind];
            grp = GemmGroup{};
            sv.loose[kind].clear();
            bool wanted = true;
            for (int64_t e = 0; e < E; ++e) wanted = expert_call(L, sv, kind, e, 0, 0, &calls[static_cast<size_t>(e)]);
            if (!wanted) continue;  // no expert's gradient of this kind is trained
            const GemmCall& g0 = calls[0];
            const bool seg = g0.seg != nullptr;
            int tile = 4;
            while (!seg && tile > 1 && E * ceil_div(g0.J, 32 * tile) * ceil_div(even, 32 * tile) < 512) tile /= 2;
            const int64_t T = 32 * tile;
            const int64_t max_tiles = seg ? E * ceil_div(g0.I, T) * ceil_div(g0.J, T)
                                          : ceil_div(g0.J, T) * (ceil_div(R * K, T) + E);
            DLLM_TRY(gemm_row_group_prepare(calls.data(), static_cast<int>(E), static_cast<int>(E), tile, max_tiles,
                                            host.data() + kind * gb, &grp));
        }
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "expert templates"));  // no fill still reads the old template
        DLLM_TRY(check_hip(hipMemcpy(sv.tmpl, host.data(), host.size(), hipMemcpyHostToDevice), "upload"));
        sv.tmpl_key = key;
        return kOk;
    }

    // Groups the layer's rows by expert on the device and writes the live tables of its expert matmuls: no host
    // round trip, so the stream keeps running through routed layers.
    int group_rows_device(int64_t l, Saved& sv, int64_t R, hipStream_t s) {
        DLLM_TRY(expert_templates(l, sv, R, s));
        DLLM_TRY(launch_moe_group_rows(sv.chosen, R, K, E, seg_d, static_cast<int>(nwin), group_cnt, sv.estart_d,
                                       sv.eseg, W_max + 1, sv.row_of, sv.slot, sv.order, pos_of, counts_d,
                                       route_err, s));
        const size_t gb = gemm_group_bytes(static_cast<int>(E));
        for (int kind = 0; kind < kExpertMatmuls; ++kind) {
            if (sv.groups[kind].count == 0) continue;
            DLLM_TRY(launch_gemm_row_group_fill(sv.tmpl + kind * gb, sv.tables + kind * gb, sv.groups[kind],
                                                sv.estart_d, expert_shift(kind), s));
        }
        if (profiling) {  // the matmul timing's algorithmic flop needs the group sizes (not a timed step)
            sv.estart.assign(static_cast<size_t>(E + 1), 0);
            DLLM_TRY(check_hip(hipMemcpyAsync(sv.estart.data(), sv.estart_d, sv.estart.size() * 8,
                                              hipMemcpyDeviceToHost, s), "download"));
            DLLM_TRY(check_hip(hipStreamSynchronize(s), "group sizes"));
            const LayerIds& L = layer_ids[static_cast<size_t>(l)];
            for (int kind = 0; kind < kExpertMatmuls; ++kind) {
                sv.group_flops[kind] = 0.0;
                for (int64_t e = 0; e < E && sv.groups[kind].count > 0; ++e) {
                    GemmCall g;
                    if (expert_call(L, sv, kind, e, sv.estart[e], sv.estart[e + 1] - sv.estart[e], &g))
                        sv.group_flops[kind] += flops_of(g);
                }
            }
        }
        return kOk;
    }

    int group_rows(int64_t l, Saved& sv, int64_t R, hipStream_t s) {
        return odd_shapes ? group_rows_host(l, sv, R, s) : group_rows_device(l, sv, R, s);
    }

    int expert_matmul(const Saved& sv, int kind, hipStream_t s) {
        if (!sv.loose[kind].empty()) {
            for (const GemmCall& g : sv.loose[kind]) DLLM_TRY(gemm(g, s));
            return kOk;
        }
        const size_t gb = gemm_group_bytes(static_cast<int>(E));
        return gemm_group(sv.groups[kind], sv.tables + kind * gb, sv.group_flops[kind], s);
    }

    // _experts (backprop.py:501-527): route, group, the SwiGLU of every expert over its rows, and
    // x_out = x_mid + sum over the row's experts (ascending) of f32(y w).
    int moe_forward(int64_t l, int64_t R, float* x_out, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        Saved& sv = saved[static_cast<size_t>(l)];
        DLLM_TRY(linear_fwd(sv.h2, R, H, L.router, nullptr, sv.router_logits, nullptr, s));
        DLLM_TRY(launch_moe_route(sv.router_logits, R, E, K, c.normalize_expert_weights ? 1 : 0, sv.chosen,
                                  sv.routing, sv.probs, s));
        DLLM_TRY(group_rows(l, sv, R, s));
        DLLM_TRY(launch_gather_rows(sv.h2, sv.row_of, xg, R * K, H, s));
        DLLM_TRY(expert_matmul(sv, kFwdGate, s));
        DLLM_TRY(expert_matmul(sv, kFwdUp, s));
        DLLM_TRY(launch_swiglu_forward(sv.gate, sv.up, sv.gate_act, sv.product, R * K * EI, s, act()));
        DLLM_TRY(expert_matmul(sv, kFwdDown, s));
        // with post norms (backprop.py:462-463) the experts' sum is the MLP output sv.mlp, normalised, then added
        if (c.shared_inter == 0) {
            if (!post_norms()) return launch_moe_combine(sv.y, sv.order, sv.slot, sv.routing, sv.x_mid, x_out, R, K, H, s);
            DLLM_TRY(launch_moe_combine(sv.y, sv.order, sv.slot, sv.routing, nullptr, sv.mlp, R, K, H, s));
            return mlp_post_norm(l, R, x_out, s);
        }
        // the shared expert over every row; out = (0 + the row's experts' f32(y w), ascending) + its (gated) output,
        // then x_out = x_mid + out (backprop.py:519-525)
        const int64_t SI = c.shared_inter;
        DLLM_TRY(linear_fwd(sv.h2, R, H, L.sgate, nullptr, sv.sh_gate, nullptr, s));
        DLLM_TRY(linear_fwd(sv.h2, R, H, L.sup, nullptr, sv.sh_up, nullptr, s));
        DLLM_TRY(launch_swiglu_forward(sv.sh_gate, sv.sh_up, sv.sh_act, sv.sh_product, R * SI, s, act()));
        DLLM_TRY(linear_fwd(sv.sh_product, R, SI, L.sdown, nullptr, sv.sh_y, nullptr, s));
        DLLM_TRY(launch_shared_gate_forward(sv.h2, L.sgw >= 0 ? P(L.sgw) : nullptr, sv.sh_y, sv.sh_s, sh_term, R, H, s));
        if (post_norms()) {
            DLLM_TRY(launch_moe_combine(sv.y, sv.order, sv.slot, sv.routing, sh_term, sv.mlp, R, K, H, s));
            return mlp_post_norm(l, R, x_out, s);
        }
        DLLM_TRY(launch_moe_combine(sv.y, sv.order, sv.slot, sv.routing, sh_term, sh_out, R, K, H, s));
        return launch_add(sv.x_mid, sh_out, x_out, R * H, s);
    }

    // x_out = x_mid + post_norm(mlp) (backprop.py:462-463)
    int mlp_post_norm(int64_t l, int64_t R, float* x_out, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        const Saved& sv = saved[static_cast<size_t>(l)];
        DLLM_TRY(launch_rms_norm(sv.mlp, P(L.mlp_post), post_tmp, R, H, c.rms_norm_eps, uo(), nullptr, s));
        return launch_add(sv.x_mid, post_tmp, x_out, R * H, s);
    }

    // _experts_backward (backprop.py:308-357): dh (dh2) from dmlp, the gradient of the layer's MLP output (dx, or
    // with post norms the gradient through the MLP's post norm).
    int moe_backward(int64_t l, int64_t R, int nseg, const float* dmlp, hipStream_t s) {
        const LayerIds& L = layer_ids[static_cast<size_t>(l)];
        const Saved& sv = saved[static_cast<size_t>(l)];
        const int64_t P = R * K;
        DLLM_TRY(launch_moe_dweights(dmlp, sv.y, sv.row_of, sv.slot, sv.routing, P, H, dweights, dyg, s));
        DLLM_TRY(launch_gather_rows(sv.h2, sv.row_of, xg, P, H, s));
        DLLM_TRY(expert_matmul(sv, kDxDown, s));
        DLLM_TRY(expert_matmul(sv, kDwDown, s));
        DLLM_TRY(launch_swiglu_backward(sv.gate, sv.up, sv.gate_act, dproduct, dgate, dup, P * EI, s, act()));
        DLLM_TRY(expert_matmul(sv, kDxGate, s));
        DLLM_TRY(expert_matmul(sv, kDwGate, s));
        DLLM_TRY(expert_matmul(sv, kDxUp, s));  // dx_gate + dx_up
        DLLM_TRY(expert_matmul(sv, kDwUp, s));
        // the router: dlogits from the routing weights' gradients (and the load-balancing loss's), then its linear
        if (router_scale_cur != 0.0)
            DLLM_TRY(launch_broadcast_window_rows(grad_row, seg_d, nseg, R, E, dprob, s));
        DLLM_TRY(launch_moe_route_backward(sv.router_logits, sv.chosen, dweights,
                                           router_scale_cur != 0.0 ? dprob : nullptr, R, E, K,
                                           c.normalize_expert_weights ? 1 : 0, dlogits_r, s));
        hipStream_t ws = s;  // dlogits_r is rewritten only after the next layer's wait on this mark
        DLLM_TRY(side_fork_from(s, &ws));
        DLLM_TRY(linear_dw(dlogits_r, E, sv.h2, H, nseg, G(L.router), nullptr, nullptr, ws));
        DLLM_TRY(side_mark(kSideMlp));
        DLLM_TRY(linear_dx(dlogits_r, R, L.router, dh2r, nullptr, s));
        // dh2 = (0 + the experts' dx in expert order) + dh2_router
        if (c.shared_inter == 0) return launch_moe_combine(dxg, sv.order, sv.slot, nullptr, dh2r, dh, R, K, H, s);
        // with a shared expert (backprop.py:339-352): dh2 = (((0 + experts' dx) + shared dx) + gate dx) + router dx
        const int64_t SI = c.shared_inter;
        const bool gated = L.sgw >= 0;
        const float* dys = dmlp;
        if (gated) {
            const bool gate_dw = grad_wanted(G(L.sgw));
            DLLM_TRY(launch_shared_gate_backward(dmlp, sv.sh_y, sv.sh_s, this->P(L.sgw), sv.h2, dsh_dy, dsh_score, nullptr,
                                                 seg_d, nseg, gate_dw ? sh_part : nullptr, R, H, s));
            if (gate_dw) DLLM_TRY(launch_segment_sums(sh_part, H, nseg, window_weights(), G(L.sgw), s));
            dys = dsh_dy;
        }
        DLLM_TRY(linear_dx(dys, R, L.sdown, dsh_product, nullptr, s));
        DLLM_TRY(launch_swiglu_backward(sv.sh_gate, sv.sh_up, sv.sh_act, dsh_product, dsh_gate, dsh_up, R * SI, s, act()));
        // the shared expert's dW with the other weight gradients (their window partial sums share one buffer): the
        // next routed layer waits for kSideMlp before rewriting dsh_dy, dsh_gate, dsh_up, and dx is kept until
        // kSideDown when the down dW reads it
        hipStream_t sws = s;
        DLLM_TRY(side_fork_from(s, &sws));
        DLLM_TRY(linear_dw(dys, H, sv.sh_product, SI, nseg, G(L.sdown), nullptr, nullptr, sws, nullptr, -1,
                           unfold_scale(L.sdown)));
        if (dys == dx) DLLM_TRY(side_mark(kSideDown));  // (with post norms the step runs on one stream)
        DLLM_TRY(linear_dw(dsh_gate, SI, sv.h2, H, nseg, G(L.sgate), nullptr, nullptr, sws));
        DLLM_TRY(linear_dw(dsh_up, SI, sv.h2, H, nseg, G(L.sup), nullptr, nullptr, sws));
        DLLM_TRY(side_mark(kSideMlp));
        DLLM_TRY(linear_dx(dsh_gate, R, L.sgate, dsh_x, nullptr, s));
        DLLM_TRY(linear_dx(dsh_up, R, L.sup, dsh_x, dsh_x, s));  // dx_gate + dx_up
        DLLM_TRY(launch_moe_combine(dxg, sv.order, sv.slot, nullptr, dsh_x, dh, R, K, H, s));
        if (gated)  // + f32(dscore w), the gate's input gradient
            DLLM_TRY(launch_shared_gate_backward(dmlp, sv.sh_y, sv.sh_s, this->P(L.sgw), sv.h2, nullptr, dsh_score, dh,
                                                 seg_d, nseg, nullptr, R, H, s));
        return launch_add(dh, dh2r, dh, R * H, s);
    }

    // Host preparation of a batch of windows; returns the packed row count.
    int prepare(const int64_t* tokens, const int64_t* offsets, const int64_t* lengths, int64_t windows, int64_t* rows_out,
                AttentionBatch* b, int64_t* groups_out, hipStream_t s) {
        DLLM_REQUIRE(windows >= 1 && windows <= W_max, "number of windows outside the trainer's capacity");
        std::vector<int64_t> in, tgt, pos, seg(1, 0), qs, ql;
        int64_t max_len = 0;
        for (int64_t w = 0; w < windows; ++w) {
            DLLM_REQUIRE(lengths[w] >= 2, "a window needs at least two tokens");
            const int64_t n = lengths[w] - 1;
            DLLM_REQUIRE(n <= T_max, "window longer than the trainer's capacity");
            qs.push_back(seg.back());
            ql.push_back(n);
            for (int64_t t = 0; t < n; ++t) {
                const int64_t a = tokens[offsets[w] + t], z = tokens[offsets[w] + t + 1];
                DLLM_REQUIRE(a >= 0 && a < V && z >= 0 && z < V, "token id out of range");
                in.push_back(a);
                tgt.push_back(ignore_targets != nullptr && t < ignore_targets[w] ? -1 : z);
                pos.push_back(t);
            }
            seg.push_back(seg.back() + n);
            max_len = std::max(max_len, n);
        }
        const int64_t R = seg.back();
        DLLM_REQUIRE(R <= R_max, "more tokens than the trainer's capacity");
        seg_host = seg;
        // embedding groups (grad.hpp:433-447 per window): rows of each window grouped by token, positions ascending
        std::vector<int64_t> order, starts, outs;
        std::vector<int> amap(static_cast<size_t>(windows * V), -1);
        for (int64_t w = 0; w < windows; ++w) {
            std::vector<int64_t> rows;
            for (int64_t r = seg[w]; r < seg[w + 1]; ++r) rows.push_back(r);
            std::stable_sort(rows.begin(), rows.end(), [&](int64_t a, int64_t z) { return in[a] < in[z]; });
            for (size_t i = 0; i < rows.size(); ++i) {
                if (i == 0 || in[rows[i]] != in[rows[i - 1]]) {
                    amap[static_cast<size_t>(w * V + in[rows[i]])] = static_cast<int>(starts.size());
                    outs.push_back(static_cast<int64_t>(starts.size()));
                    starts.push_back(static_cast<int64_t>(order.size()));
                }
                order.push_back(rows[i]);
            }
        }
        starts.push_back(static_cast<int64_t>(order.size()));
        std::vector<int64_t> batch(qs);
        batch.insert(batch.end(), ql.begin(), ql.end());
        batch.insert(batch.end(), qs.begin(), qs.end());
        batch.insert(batch.end(), ql.begin(), ql.end());
        // the step's inputs through the pinned staging buffer, copied on the stream (the previous step, which read
        // the device copies and the staging buffer, has been waited for)
        size_t staged = 0;
        auto upload = [&](void* dst, const void* src, size_t bytes) -> int {
            DLLM_REQUIRE(staged + bytes <= staging_bytes, "step inputs exceed the staging buffer");
            memcpy(staging + staged, src, bytes);
            const int rc = check_hip(hipMemcpyAsync(dst, staging + staged, bytes, hipMemcpyHostToDevice, s), "upload");
            staged += (bytes + 255) & ~size_t{255};
            return rc;
        };
        DLLM_TRY(upload(tok_in, in.data(), R * 8));
        DLLM_TRY(upload(tok_tgt, tgt.data(), R * 8));
        DLLM_TRY(upload(pos_index, pos.data(), R * 8));
        DLLM_TRY(upload(seg_d, seg.data(), seg.size() * 8));
        DLLM_TRY(upload(batch_d, batch.data(), batch.size() * 8));
        DLLM_TRY(upload(grp_order, order.data(), order.size() * 8));
        DLLM_TRY(upload(grp_start, starts.data(), starts.size() * 8));
        DLLM_TRY(upload(grp_out, outs.data(), outs.size() * 8));
        DLLM_TRY(upload(addrow, amap.data(), amap.size() * sizeof(int)));
        b->q_start = batch_d;
        b->q_len = batch_d + windows;
        b->kv_start = batch_d + 2 * windows;
        b->kv_len = batch_d + 3 * windows;
        b->count = static_cast<int>(windows);
        b->max_q = max_len;
        b->max_kv = max_len;
        *rows_out = R;
        *groups_out = static_cast<int64_t>(outs.size());
        (void)s;
        return kOk;
    }

    int gradients(const int64_t* tokens, const int64_t* offsets, const int64_t* lengths, int64_t windows,
                  double scale, double router_scale, double* loss, double* router_loss, hipStream_t s) {
        int64_t R = 0, groups = 0;
        AttentionBatch b{};
        DLLM_TRY(prepare(tokens, offsets, lengths, windows, &R, &b, &groups, s));
        if (lora_on) {
            DLLM_TRY(prepare_lora(s));
        } else if (!wt_valid) {
            if (fold_on) DLLM_TRY(fold_weights(s));
            DLLM_TRY(refresh_transposes(s));
        }
        DLLM_TRY(prepare_groups(R, s));
        const int nseg = static_cast<int>(windows);
        nwin = windows;
        router_scale_cur = router_scale;
        if (E > 0) {  // the router statistics' per-window choice counts, summed over the sparse layers
            counts_host.assign(static_cast<size_t>(windows * E), 0);
            if (!odd_shapes) DLLM_TRY(launch_zero_i64(counts_d, windows * E, s));
            DLLM_TRY(check_hip(hipMemsetAsync(route_err, 0, sizeof(int), s), "memset"));
        }
        const double eps = c.rms_norm_eps;
        // forward (backprop.py:411-490)
        DLLM_TRY(launch_gather_rows(P(emb), tok_in, saved[0].x_in, R, H, s));
        if (c.embedding_multiplier != 1.0)
            DLLM_TRY(launch_scale(saved[0].x_in, R * H, static_cast<float>(c.embedding_multiplier), false, s));
        for (int64_t l = 0; l < c.layers; ++l) {
            float* x_out = l + 1 < c.layers ? saved[static_cast<size_t>(l + 1)].x_in : x_final;
            DLLM_TRY(forward_layer(l, R, b, x_out, s));
        }
        if (E > 0) {  // _router_loss (backprop.py:359-377): per window, over every sparse layer's rows
            if (odd_shapes)  // host grouping counted them on the host
                DLLM_TRY(check_hip(hipMemcpyAsync(counts_d, counts_host.data(), counts_host.size() * 8,
                                                  hipMemcpyHostToDevice, s), "upload"));
            DLLM_TRY(launch_router_stats(probs_all, R_max * E, sparse_layers(), seg_d, nseg, counts_d, E, router_scale,
                                         router_loss_w, router_scale != 0.0 ? grad_row : nullptr, s));
        }
        DLLM_TRY(launch_rms_norm(x_final, P(final_norm), hidden, R, H, eps, uo(), nullptr, s));
        const int head = c.tie_embeddings ? emb : lm_head;
        DLLM_TRY(linear_fwd(hidden, R, H, head, nullptr, logits, nullptr, s));
        // loss and the head (backprop.py:174-206): Granite's logits scaling divides the logits and their gradient
        const bool logit_div = c.logits_scaling != 1.0;
        if (logit_div) DLLM_TRY(launch_scale(logits, R * V, static_cast<float>(c.logits_scaling), true, s));
        DLLM_TRY(check_hip(hipMemsetAsync(err_flag, 0, sizeof(int), s), "memset"));
        if (c.logits_softcap != 0.0) DLLM_TRY(launch_softcap(logits, logits_capped, R * V, c.logits_softcap, s));
        DLLM_TRY(launch_cross_entropy(c.logits_softcap != 0.0 ? logits_capped : logits, tok_tgt, dlogits, R, V, scale,
                                      seg_d, nseg, row_max, row_total, row_loss, loss_w, err_flag, s));
        if (c.logits_softcap != 0.0)
            DLLM_TRY(launch_softcap_backward(logits, dlogits, dlogits, R * V, c.logits_softcap, s));
        if (logit_div) DLLM_TRY(launch_scale(dlogits, R * V, static_cast<float>(c.logits_scaling), true, s));
        if (dpo.on) DLLM_TRY(dpo_weights(windows, s));
        float* dhidden = dh;
        DLLM_TRY(linear_dx(dlogits, R, head, dhidden, nullptr, s));
        DLLM_TRY(launch_rms_norm_backward_dx(x_final, P(final_norm), dhidden, dx, nullptr, R, H, eps, uo(), inv_rms, s));
        DLLM_TRY(norm_dw(dhidden, x_final, inv_rms, H, 1, nseg, G(final_norm), s));
        for (bool& pending : side_pending) pending = false;
        side_on = false;
        if (!profiling && !post_norms() && !odd_shapes) {  // the post norms' buffers (and the matmul scratch) are
                                                              // ordered by the one stream
            DLLM_TRY(side_setup());
            side_on = true;
        }
        for (int64_t l = c.layers - 1; l >= 0; --l) DLLM_TRY(backward_layer(l, R, nseg, b, s));
        DLLM_TRY(side_join(s));
        // embedding (backprop.py:112-117): per-window token rows, then the head's dW with them as the tied addend
        if (lora_on) return finish_gradients(windows, loss, router_loss, s);  // neither is adapted
        if (c.embedding_multiplier != 1.0)  // backprop.py:110-111
            DLLM_TRY(launch_scale(dx, R * H, static_cast<float>(c.embedding_multiplier), false, s));
        DLLM_TRY(launch_embedding_groups(dx, H, grp_order, grp_start, grp_out, groups, emb_rows, H, s));
        if (c.tie_embeddings) {
            DLLM_TRY(linear_dw(dlogits, V, hidden, H, nseg, G(emb), addrow, emb_rows, s));
        } else {
            DLLM_TRY(linear_dw(dlogits, V, hidden, H, nseg, G(lm_head), nullptr, nullptr, s));
            hipLaunchKernelGGL(sparse_window_sum_kernel, dim3(static_cast<unsigned>(V)), dim3(256), 0, s, emb_rows,
                               addrow, V, H, nseg, window_weights(), G(emb));
            DLLM_TRY(check_launch("embedding window sum"));
        }
        return finish_gradients(windows, loss, router_loss, s);
    }

    // The losses of the step's windows, summed in window order on the host.
    int finish_gradients(int64_t windows, double* loss, double* router_loss, hipStream_t s) {
        std::vector<double> lw(static_cast<size_t>(windows)), rw(static_cast<size_t>(windows), 0.0);
        int flag = 0;
        DLLM_TRY(check_hip(hipMemcpyAsync(lw.data(), loss_w, lw.size() * 8, hipMemcpyDeviceToHost, s), "download"));
        if (E > 0)
            DLLM_TRY(check_hip(hipMemcpyAsync(rw.data(), router_loss_w, rw.size() * 8, hipMemcpyDeviceToHost, s),
                               "download"));
        DLLM_TRY(check_hip(hipMemcpyAsync(&flag, err_flag, sizeof flag, hipMemcpyDeviceToHost, s), "download"));
        int route_flag = 0;
        if (E > 0)
            DLLM_TRY(check_hip(hipMemcpyAsync(&route_flag, route_err, sizeof route_flag, hipMemcpyDeviceToHost, s),
                               "download"));
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "step"));
        DLLM_REQUIRE(flag == 0, "target out of range");
        DLLM_REQUIRE(route_flag == 0, "routing produced an expert out of range");
        window_losses = lw;
        double total = 0.0;
        for (double x : lw) total += x;  // trainer.py:326 (loss_total += loss, batch order)
        if (loss) *loss = total;
        double rtotal = 0.0;
        for (double x : rw) rtotal += x;  // trainer.py:327 (router_total += router_loss, batch order)
        last_router_loss = rtotal;
        if (router_loss) *router_loss = rtotal;
        return kOk;
    }

    int step(const int64_t* tokens, const int64_t* offsets, const int64_t* lengths, int64_t windows,
             const dllm_hip_adamw* a, double* loss, double* norm, hipStream_t s) {
        int64_t targets_total = 0;
        for (int64_t w = 0; w < windows; ++w) targets_total += lengths[w] - 1;
        DLLM_REQUIRE(targets_total > 0, "a step needs targets");
        const double scale = 1.0 / static_cast<double>(targets_total);
        double loss_total = 0.0, router_total = 0.0;
        DLLM_TRY(gradients(tokens, offsets, lengths, windows, scale, a->router_aux_loss / static_cast<double>(windows),
                           &loss_total, &router_total, s));
        double grad_norm = 0.0;
        DLLM_TRY(optimizer_step(a, &grad_norm, s));
        if (loss) {
            *loss = loss_total / static_cast<double>(targets_total);
            if (a->router_aux_loss != 0.0)  // trainer.py:333-335
                *loss += a->router_aux_loss * router_total / static_cast<double>(windows);
        }
        if (norm) *norm = grad_norm;
        return kOk;
    }

    // The update of a step from its summed gradients (trainer.py:303-306): LoRA adapter gradients, the global norm and
    // clip, and AdamW over what the run trains (waits; *norm gets the norm before clipping).
    int optimizer_step(const dllm_hip_adamw* a, double* norm, hipStream_t s) {
        if (lora_on) DLLM_TRY(adapter_gradients(s));  // trainer.py:463-474
        OptimizerSet& o = lora_on ? lora_opt : main_opt;
        // global norm, clip (optimizer.py:66-90), bias corrections by repeated multiplication (optimizer.py:59-63)
        DLLM_TRY(launch_exact_sum_squares(o.g, o.norm_plan, o.norm_ws, o.per_tensor, s));
        DLLM_TRY(launch_norm_finish(o.per_tensor, o.tensors, a->max_grad_norm, stats, s));
        double p1 = 1.0, p2 = 1.0;
        for (int64_t i = 0; i < a->step; ++i) {
            p1 *= a->beta1;
            p2 *= a->beta2;
        }
        AdamWArgs args{a->learning_rate, a->beta1, a->beta2, a->eps, 1.0 - p1, 1.0 - p2, 1.0};
        // the chunk table holds 1 for matrices: decay = weight_decay * 1 or * 0 (optimizer.py:93)
        DLLM_TRY(scale_decay(o, a->weight_decay));
        DLLM_TRY(launch_adamw(o.p, o.g, o.m, o.v, o.chunk_start, o.chunk_end, o.chunk_decay_scaled, o.chunks, args,
                              stats + 2, s));
        if (lora_on) {
            merged_valid = false;  // the next step merges the updated adapters
        } else {
            if (fold_on) DLLM_TRY(fold_weights(s));  // the folded copies of the updated q/k rows (or QK-norm weights)
            DLLM_TRY(refresh_transposes(s));
        }
        double st[3];
        DLLM_TRY(check_hip(hipMemcpyAsync(st, stats, sizeof st, hipMemcpyDeviceToHost, s), "download"));
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "step"));
        *norm = st[1];
        return kOk;
    }

    // ---- direct preference optimization (trainer.py:364-384, preference.py:166-179) ----
    // Windows 2p and 2p + 1 are pair p's chosen and rejected sequences; their targets over the prompt are ignored, so
    // each window's summed cross-entropy is minus its answer's log-probability. Once the forward pass has the window
    // losses, the host computes every pair's z and weight; each window's gradient is then multiplied by its factor
    // (w for the chosen, -w for the rejected answer) before the window-ordered float sum, as
    // `gradients[name] += gradient * sign` does.
    struct Dpo {
        bool on = false;
        int64_t pairs = 0;
        double beta = 0.0;
        const double* reference = nullptr;  // [pairs][2]: the reference model's chosen and rejected log-probabilities
        double loss_total = 0.0;
    } dpo;
    const int64_t* ignore_targets = nullptr;  // per window: leading targets ignored (-1), or null
    float* win_weight = nullptr;
    std::vector<double> window_losses;  // the last call's per-window summed cross-entropy

    const float* window_weights() const { return dpo.on ? win_weight : nullptr; }

    static double log_sigmoid(double z) {  // preference.py:174-179 with the portable exp and log
        if (z >= 0.0) return -dlog(1.0 + dexp(-z));
        return z - dlog(1.0 + dexp(z));
    }

    int dpo_weights(int64_t windows, hipStream_t s) {
        std::vector<double> lw(static_cast<size_t>(windows));
        DLLM_TRY(check_hip(hipMemcpyAsync(lw.data(), loss_w, lw.size() * 8, hipMemcpyDeviceToHost, s), "download"));
        DLLM_TRY(check_hip(hipStreamSynchronize(s), "dpo losses"));
        std::vector<float> w(static_cast<size_t>(windows));
        dpo.loss_total = 0.0;
        for (int64_t p = 0; p < dpo.pairs; ++p) {
            const double chosen_loss = lw[static_cast<size_t>(2 * p)], rejected_loss = lw[static_cast<size_t>(2 * p + 1)];
            const double rc = dpo.reference[2 * p], rr = dpo.reference[2 * p + 1];
            const double z = dpo.beta * ((-chosen_loss - rc) - (-rejected_loss - rr));
            dpo.loss_total += -log_sigmoid(z);
            const float weight = static_cast<float>(dpo.beta * (1.0 - dsigmoid(z)) / static_cast<double>(dpo.pairs));
            w[static_cast<size_t>(2 * p)] = weight;
            w[static_cast<size_t>(2 * p + 1)] = -weight;
        }
        return check_hip(hipMemcpyAsync(win_weight, w.data(), w.size() * sizeof(float), hipMemcpyHostToDevice, s),
                         "upload");
    }

    int dpo_step(const int64_t* tokens, const int64_t* offsets, const int64_t* lengths, const int64_t* prompt_lengths,
                 int64_t pairs, const double* reference, double beta, const dllm_hip_adamw* a, double* loss,
                 double* norm, hipStream_t s) {
        DLLM_REQUIRE(pairs >= 1 && 2 * pairs <= W_max, "pairs outside the trainer's capacity");
        DLLM_REQUIRE(beta > 0.0 && beta < HUGE_VAL, "beta must be a positive number");
        std::vector<int64_t> ignore(static_cast<size_t>(2 * pairs));
        for (int64_t p = 0; p < pairs; ++p) {
            DLLM_REQUIRE(prompt_lengths[p] >= 1, "a pair needs a prompt");
            for (int k = 0; k < 2; ++k) {
                DLLM_REQUIRE(lengths[2 * p + k] > prompt_lengths[p], "an answer is empty");
                ignore[static_cast<size_t>(2 * p + k)] = prompt_lengths[p] - 1;
            }
        }
        dpo = Dpo{true, pairs, beta, reference, 0.0};
        ignore_targets = ignore.data();
        const int status = gradients(tokens, offsets, lengths, 2 * pairs, 1.0, 0.0, nullptr, nullptr, s);
        ignore_targets = nullptr;
        dpo.on = false;
        DLLM_TRY(status);
        double grad_norm = 0.0;
        DLLM_TRY(optimizer_step(a, &grad_norm, s));
        if (loss) *loss = dpo.loss_total / static_cast<double>(pairs);  // trainer.py:384
        if (norm) *norm = grad_norm;
        return kOk;
    }

    // Minus the summed cross-entropy of each window with the leading targets ignored: the answers' log-probabilities
    // (FineTuner.log_probability, trainer.py:443-453; the gradients are computed and not used).
    int log_probabilities(const int64_t* tokens, const int64_t* offsets, const int64_t* lengths,
                          const int64_t* prompt_lengths, int64_t windows, double* out, hipStream_t s) {
        std::vector<int64_t> ignore(static_cast<size_t>(windows));
        for (int64_t w = 0; w < windows; ++w) {
            DLLM_REQUIRE(prompt_lengths[w] >= 1 && lengths[w] > prompt_lengths[w], "a window needs a prompt and an answer");
            ignore[static_cast<size_t>(w)] = prompt_lengths[w] - 1;
        }
        ignore_targets = ignore.data();
        const int status = gradients(tokens, offsets, lengths, windows, 1.0, 0.0, nullptr, nullptr, s);
        ignore_targets = nullptr;
        DLLM_TRY(status);
        for (int64_t w = 0; w < windows; ++w) out[w] = -window_losses[static_cast<size_t>(w)];
        return kOk;
    }

    int scale_decay(OptimizerSet& o, double wd) {
        if (wd == o.last_decay) return kOk;
        std::vector<double> d(static_cast<size_t>(o.chunks));
        if (!d.empty()) {
            DLLM_TRY(check_hip(hipMemcpy(d.data(), o.chunk_decay, d.size() * 8, hipMemcpyDeviceToHost), "download"));
            for (double& x : d) x = x != 0.0 ? wd : 0.0;
            DLLM_TRY(check_hip(hipMemcpy(o.chunk_decay_scaled, d.data(), d.size() * 8, hipMemcpyHostToDevice), "upload"));
        }
        o.last_decay = wd;
        return kOk;
    }

    // ---- LoRA (lora.py) ----
    bool merged_valid = false;

    // The adapted weights (target_weights, lora.py:211-242): q k v o gate up down by the target mask.
    int build_lora(const dllm_hip_lora_config& l) {
        lora_on = true;
        lc = l;
        lora_scale = static_cast<float>(l.alpha / (l.rslora ? std::sqrt(static_cast<double>(l.rank))
                                                           : static_cast<double>(l.rank)));
        static const char* kTargets[7] = {"attention.q.weight", "attention.k.weight", "attention.v.weight",
                                          "attention.o.weight", "mlp.gate.weight", "mlp.up.weight",
                                          "mlp.down.weight"};
        std::vector<int> weights;
        for (int64_t layer = 0; layer < c.layers; ++layer)
            for (int t = 0; t < 7; ++t) {
                if (!(l.targets & (int64_t{1} << t))) continue;
                const LayerIds& L = layer_ids[static_cast<size_t>(layer)];
                if (t >= 4 && sparse(layer)) {  // gate, up, down of a routed layer: every expert's (the router never)
                    const std::vector<int>& ids = t == 4 ? L.egate : (t == 5 ? L.eup : L.edown);
                    weights.insert(weights.end(), ids.begin(), ids.end());
                    const int shared = t == 4 ? L.sgate : (t == 5 ? L.sup : L.sdown);  // and the shared expert's
                    if (shared >= 0) weights.push_back(shared);
                } else {
                    weights.push_back(index["layers." + std::to_string(layer) + "." + kTargets[t]]);
                }
            }
        for (int w : weights) {
            const TensorInfo& t = tensors[static_cast<size_t>(w)];
            TensorInfo a, b;
            a.name = t.name + ".lora_a";
            a.rows = l.rank;
            a.cols = t.cols;
            b.name = t.name + ".lora_b";
            b.rows = t.rows;
            b.cols = l.rank;
            a.ndim = b.ndim = 2;
            a.numel = a.rows * a.cols;
            b.numel = b.rows * b.cols;
            adapters.push_back(a);
            adapters.push_back(b);
        }
        std::stable_sort(adapters.begin(), adapters.end(),
                         [](const TensorInfo& x, const TensorInfo& y) { return natural_less(x.name, y.name); });
        int64_t off = 0;
        for (size_t i = 0; i < adapters.size(); ++i) {
            off = static_cast<int64_t>(round_up(static_cast<size_t>(off), 64));
            adapters[i].offset = off;
            off += adapters[i].numel;
            adapter_index[adapters[i].name] = static_cast<int>(i);
        }
        const size_t arena = static_cast<size_t>(round_up(static_cast<size_t>(off > 0 ? off : 1), 64)) * sizeof(float);
        for (DevBuf* d : {&lora_p, &lora_g, &lora_m, &lora_v}) {
            DLLM_TRY(d->alloc(arena));
            DLLM_TRY(check_hip(hipMemset(d->p, 0, arena), "memset"));
        }
        int64_t moff = 0;
        size_t ws = 0;
        int64_t largest = 0;
        for (int w : weights) {
            const TensorInfo& t = tensors[static_cast<size_t>(w)];
            moff = static_cast<int64_t>(round_up(static_cast<size_t>(moff), 64));
            merged_offset[static_cast<size_t>(w)] = moff;
            moff += t.numel;
            lora_targets.push_back({w, adapter_index[t.name + ".lora_a"], adapter_index[t.name + ".lora_b"]});
            target_grads.push_back(G(w));
            ws = std::max(ws, lora_merge_workspace(t.rows, t.cols, l.rank));
            ws = std::max(ws, lora_adapter_gradients_workspace(t.rows, t.cols, l.rank));
        }
        for (const TensorInfo& t : tensors)
            if (quantizable(t)) largest = std::max(largest, t.numel);
        DLLM_TRY(merged.alloc(static_cast<size_t>(moff > 0 ? moff : 1) * sizeof(float)));
        char* w = nullptr;
        DLLM_TRY(make(&w, std::max<size_t>(ws, 1)));
        lora_ws = w;
        lora_ws_bytes = std::max<size_t>(ws, 1);
        if (l.base_quantize) {
            DLLM_TRY(make(&q8_values, static_cast<size_t>(std::max<int64_t>(largest, 32))));
            DLLM_TRY(make(&q8_scales, static_cast<size_t>(std::max<int64_t>(largest / 32, 1))));
            if (l.base_quantize == 2) DLLM_TRY(make(&q4_packed, static_cast<size_t>(std::max<int64_t>(largest / 2, 16))));
            base_ready = false;
        }
        return build_optimizer(adapters, lora_p.as<float>(), lora_g.as<float>(), lora_m.as<float>(),
                               lora_v.as<float>(), &lora_opt);
    }

    // quantizable (lora.py:300-302): the q k v o gate up down matrices whose input size is a multiple of 32
    static bool quantizable(const TensorInfo& t) {
        static const char* kSuffix[7] = {".q.weight", ".k.weight", ".v.weight", ".o.weight", ".gate.weight",
                                         ".up.weight", ".down.weight"};
        if (t.ndim != 2 || t.cols % 32 != 0) return false;
        for (const char* sfx : kSuffix) {
            const size_t n = strlen(sfx);
            if (t.name.size() > n && t.name.compare(t.name.size() - n, n, sfx) == 0) return true;
        }
        return false;
    }

    // Before a step: the quantised base once per parameter write (QuantizedBase: reading a quantised matrix gives its
    // dequantised values, int8 value times block scale in float32 for Q8_0 and for unpacked Q4_0 alike,
    // numerics.py:131-139), then W' = merge(W, A, B) for every target (lora.py:271-287) and their W'^T.
    int prepare_lora(hipStream_t s) {
        if (!base_ready) {
            for (const TensorInfo& t : tensors) {
                if (!quantizable(t)) continue;
                float* w = params.as<float>() + t.offset;
                if (lc.base_quantize == 2) {
                    DLLM_TRY(dllm_hip_quantize_q4_0(w, q4_packed, q8_scales, static_cast<size_t>(t.numel), s));
                    DLLM_TRY(dllm_hip_unpack_q4_0(q4_packed, q8_values, static_cast<size_t>(t.numel), s));
                } else {
                    DLLM_TRY(launch_quantize_q8_0(w, q8_values, q8_scales, t.numel, s));
                }
                DLLM_TRY(launch_dequantize_q8_0(q8_values, q8_scales, w, t.numel, s));
            }
            base_ready = true;
            wt_valid = false;
            merged_valid = false;
        }
        if (merged_valid && wt_valid) return kOk;
        for (const LoraTarget& lt : lora_targets) {
            const TensorInfo& t = tensors[static_cast<size_t>(lt.weight)];
            DLLM_TRY(launch_lora_merge(params.as<float>() + t.offset, lora_p.as<float>() + adapters[lt.a].offset,
                                       lora_p.as<float>() + adapters[lt.b].offset,
                                       merged.as<float>() + merged_offset[static_cast<size_t>(lt.weight)], t.rows,
                                       t.cols, lc.rank, lora_scale, lora_ws, lora_ws_bytes, s));
        }
        merged_valid = true;
        if (fold_on) DLLM_TRY(fold_weights(s));
        return refresh_transposes(s);
    }

    // dA, dB of every target from the merged weight's gradient (trainer.py:463-474, lora.py:374-383).
    int adapter_gradients(hipStream_t s) {
        for (const LoraTarget& lt : lora_targets) {
            const TensorInfo& t = tensors[static_cast<size_t>(lt.weight)];
            DLLM_TRY(launch_lora_adapter_gradients(G(lt.weight), lora_p.as<float>() + adapters[lt.a].offset,
                                                   lora_p.as<float>() + adapters[lt.b].offset,
                                                   lora_g.as<float>() + adapters[lt.a].offset,
                                                   lora_g.as<float>() + adapters[lt.b].offset, t.rows, t.cols,
                                                   lc.rank, lora_scale, lora_ws, lora_ws_bytes, s));
        }
        return kOk;
    }

    // The data sections of the reference's files (device pointers, in file order):
    //   kModelFile: weights() in natural order (trainer.py:460-468): the parameters, with every LoRA target merged
    //     (and a Q8_0 base applied), as FineTuner.export writes them (trainer.py:477-509);
    //   kCheckpointFile: _checkpoint_tensors (trainer.py:519-522): "param/<name>" for the trained tensors (the
    //     adapters in a LoRA run) in natural order, then adam_m/<name>, adam_v/<name> per tensor in natural order
    //     (optimizer.py:111-114).
    int file_tensors(int kind, std::vector<TensorSource>* out, hipStream_t s) {
        out->clear();
        if (kind == kModelFile) {
            if (lora_on) DLLM_TRY(prepare_lora(s));
            for (size_t i = 0; i < tensors.size(); ++i) {
                const TensorInfo& t = tensors[i];
                const bool merged_t = lora_on && merged_offset[i] >= 0;
                out->push_back(TensorSource{(merged_t ? merged.as<float>() + merged_offset[i] : params.as<float>() +
                                                                                                      t.offset),
                                            t.numel, true});
            }
            return kOk;
        }
        const std::vector<TensorInfo>& set = lora_on ? adapters : tensors;
        const DevBuf& p = lora_on ? lora_p : params;
        const DevBuf& m = lora_on ? lora_m : m1;
        const DevBuf& v = lora_on ? lora_v : m2;
        for (const TensorInfo& t : set) out->push_back(TensorSource{p.as<float>() + t.offset, t.numel, true});
        for (const TensorInfo& t : set) {
            out->push_back(TensorSource{m.as<float>() + t.offset, t.numel, true});
            out->push_back(TensorSource{v.as<float>() + t.offset, t.numel, true});
        }
        return kOk;
    }
};

extern "C" {

int dllm_hip_trainer_create_lora(const dllm_hip_decoder_config* config, const dllm_hip_lora_config* lora,
                                 int64_t max_tokens, int64_t max_windows, int64_t max_window_tokens,
                                 dllm_hip_trainer** out) {
    DLLM_REQUIRE(config && out, "null argument");
    if (lora) {
        DLLM_REQUIRE(lora->rank >= 1, "the LoRA rank must be positive");
        DLLM_REQUIRE(lora->targets > 0 && lora->targets < 128, "LoRA targets must be a non-empty subset of q k v o gate up down");
        DLLM_REQUIRE(lora->base_quantize >= 0 && lora->base_quantize <= 2,
                     "base_quantize must be 0 (float), 1 (q8_0) or 2 (q4_0)");
    }
    const dllm_hip_decoder_config& c = *config;
    const int64_t ei = c.experts > 0 ? (c.expert_intermediate > 0 ? c.expert_intermediate : c.intermediate) : 0;
    DLLM_REQUIRE(c.experts >= 0, "negative number of experts");
    if (c.experts > 0) {
        DLLM_REQUIRE(c.experts_per_token >= 1 && c.experts_per_token <= c.experts,
                     "experts per token must be between 1 and the number of experts");
        DLLM_REQUIRE(ei > 0, "the expert intermediate size must be positive");
    }
    DLLM_REQUIRE(c.heads > 0 && c.kv_heads > 0 && c.heads % c.kv_heads == 0, "heads must be a multiple of kv_heads");
    DLLM_REQUIRE(c.rotary_dim > 0 && c.rotary_dim % 2 == 0 && c.rotary_dim <= c.head_dim, "invalid rotary_dim");
    DLLM_REQUIRE(c.head_dim % 4 == 0, "head_dim must be a multiple of 4 (the attention tiles' 16-byte operand rows)");
    DLLM_REQUIRE(c.vocab > 0 && c.hidden > 0 && c.intermediate > 0 && c.layers > 0, "sizes must be positive");
    DLLM_REQUIRE(max_tokens > 0 && max_windows > 0 && max_window_tokens > 0, "capacities must be positive");
    // the attention chains run one workgroup row per (window, head) in the grid's second dimension
    DLLM_REQUIRE(max_windows * c.heads <= 65535, "at most 65535 (window, head) pairs per step");
    for (double m : {c.embedding_multiplier, c.residual_multiplier, c.logits_scaling})
        DLLM_REQUIRE(m >= 0.0 && std::isfinite(m), "multipliers must be finite and non-negative (0: none)");
    DLLM_REQUIRE(c.attention_scale > 0.0 && std::isfinite(c.attention_scale), "attention_scale must be positive");
    DLLM_REQUIRE(c.norm_placement >= 0 && c.norm_placement <= 2, "norm_placement must be 0 (pre), 1 (post) or 2 (both)");
    DLLM_REQUIRE(c.shared_inter >= 0, "the shared expert's size must not be negative");
    DLLM_REQUIRE(c.shared_inter == 0 || c.experts > 0, "a shared expert needs routed experts");
    DLLM_REQUIRE(c.shared_gate == 0 || c.shared_inter > 0, "a shared expert gate needs a shared expert");
    DLLM_REQUIRE(c.activation == 0 || c.activation == 1, "activation must be 0 (silu) or 1 (gelu_tanh)");
    DLLM_REQUIRE(c.local_rope_theta >= 0.0 && c.attention_softcap >= 0.0 && c.logits_softcap >= 0.0,
                 "local_rope_theta and the soft-caps must be non-negative (0: none)");
    std::vector<char> dense(static_cast<size_t>(c.layers)), full(static_cast<size_t>(c.layers));
    for (int64_t l = 0; l < c.layers; ++l) {
        dense[static_cast<size_t>(l)] = c.dense_layer_flags ? c.dense_layer_flags[l] != 0
                                                            : l < 64 && ((c.dense_layers >> l) & 1);
        full[static_cast<size_t>(l)] = c.full_attention_layer_flags ? c.full_attention_layer_flags[l] != 0
                                                                    : l < 64 && ((c.full_attention_layers >> l) & 1);
    }
    if (c.experts > 0) {
        bool any_sparse = false;
        for (char d : dense) any_sparse = any_sparse || !d;
        DLLM_REQUIRE(any_sparse, "a model with experts needs at least one sparse layer");
    } else {
        for (char d : dense) DLLM_REQUIRE(!d, "dense_layers needs experts");
    }
    std::unique_ptr<dllm_hip_trainer> t(new dllm_hip_trainer());
    t->c = c;
    t->c.dense_layer_flags = t->c.full_attention_layer_flags = nullptr;  // the caller's arrays are not kept
    t->dense_flag = dense;
    t->full_flag = full;
    for (double* m : {&t->c.embedding_multiplier, &t->c.residual_multiplier, &t->c.logits_scaling})
        if (*m == 0.0) *m = 1.0;  // unset
    t->R_max = max_tokens;
    t->W_max = max_windows;
    t->T_max = max_window_tokens;
    t->H = c.hidden;
    t->QD = c.heads * c.head_dim;
    t->KVD = c.kv_heads * c.head_dim;
    t->I = c.intermediate;
    t->V = c.vocab;
    t->E = c.experts;
    t->K = c.experts > 0 ? c.experts_per_token : 0;
    t->EI = ei;
    t->RK = max_tokens * t->K;
    DLLM_TRY(t->build_tensors());
    if (lora) DLLM_TRY(t->build_lora(*lora));
    DLLM_TRY(t->build_activations());
    if (t->residual_on()) {
        DLLM_TRY(t->make(&t->resid_rowscale, static_cast<size_t>(t->H)));
        const std::vector<float> rs(static_cast<size_t>(t->H), static_cast<float>(t->c.residual_multiplier));
        DLLM_TRY(check_hip(hipMemcpy(t->resid_rowscale, rs.data(), rs.size() * sizeof(float), hipMemcpyHostToDevice),
                           "upload"));
        DLLM_TRY(t->setup_fold());
    }
    *out = t.release();
    return kOk;
}

int dllm_hip_trainer_create(const dllm_hip_decoder_config* config, int64_t max_tokens, int64_t max_windows,
                            int64_t max_window_tokens, dllm_hip_trainer** out) {
    return dllm_hip_trainer_create_lora(config, nullptr, max_tokens, max_windows, max_window_tokens, out);
}

int dllm_hip_trainer_destroy(dllm_hip_trainer* t) {
    if (t) {
        (void)hipDeviceSynchronize();
        for (hipEvent_t e : t->events) (void)hipEventDestroy(e);
        if (t->staging) (void)hipHostFree(t->staging);
        if (t->side) {
            (void)hipEventDestroy(t->side_fork);
            for (hipEvent_t e : t->side_done) (void)hipEventDestroy(e);
            (void)hipStreamDestroy(t->side);
            (void)hipEventDestroy(t->aux_fork);
            (void)hipEventDestroy(t->aux_done);
            (void)hipStreamDestroy(t->aux);
        }
    }
    delete t;
    return kOk;
}

int dllm_hip_trainer_profile(dllm_hip_trainer* t, int enable) {
    DLLM_REQUIRE(t, "null argument");
    DLLM_TRY(t->drain_events());
    t->profiling = enable != 0;
    if (t->profiling) {
        t->profile_flops = 0.0;
        t->profile_launches = 0;
        t->profile_ms_done = 0.0;
    }
    return kOk;
}

int dllm_hip_trainer_profile_read(dllm_hip_trainer* t, int64_t* launches, double* ms, double* flops) {
    DLLM_REQUIRE(t, "null argument");
    DLLM_TRY(t->drain_events());
    if (launches) *launches = t->profile_launches;
    if (ms) *ms = t->profile_ms_done;
    if (flops) *flops = t->profile_flops;
    return kOk;
}

int dllm_hip_trainer_tensor(dllm_hip_trainer* t, const char* name, int which, float** ptr, int64_t* numel) {
    DLLM_REQUIRE(t && name && ptr, "null argument");
    DLLM_REQUIRE(which >= 0 && which < 4, "which must be 0 (parameter), 1 (gradient), 2 (m) or 3 (v)");
    auto ad = t->adapter_index.find(name);
    if (ad != t->adapter_index.end()) {  // a LoRA adapter: the parameters AdamW updates
        const TensorInfo& info = t->adapters[static_cast<size_t>(ad->second)];
        const DevBuf* arenas[4] = {&t->lora_p, &t->lora_g, &t->lora_m, &t->lora_v};
        *ptr = arenas[which]->as<float>() + info.offset;
        if (numel) *numel = info.numel;
        if (which == 0) t->merged_valid = false;
        return kOk;
    }
    auto it = t->index.find(name);
    DLLM_REQUIRE(it != t->index.end(), std::string("unknown tensor ") + name);
    const TensorInfo& info = t->tensors[static_cast<size_t>(it->second)];
    const DevBuf* arenas[4] = {&t->params, &t->grads, &t->m1, &t->m2};
    DLLM_REQUIRE(which >= 0 && which < 4, "which must be 0 (parameter), 1 (gradient), 2 (m) or 3 (v)");
    *ptr = arenas[which]->as<float>() + info.offset;
    if (numel) *numel = info.numel;
    if (which == 0) {  // the caller may write parameters
        t->wt_valid = false;
        t->merged_valid = false;
        if (t->lora_on && t->lc.base_quantize) t->base_ready = false;
    }
    return kOk;
}

int dllm_hip_trainer_set_rope(dllm_hip_trainer* t, const double* inv_freq, int64_t pairs, double attention_factor) {
    DLLM_REQUIRE(t && inv_freq, "null argument");
    return t->set_rope(inv_freq, pairs, attention_factor);
}

int dllm_hip_trainer_tensor_count(dllm_hip_trainer* t, int64_t* count) {
    DLLM_REQUIRE(t && count, "null argument");
    *count = static_cast<int64_t>(t->tensors.size() + t->adapters.size());
    return kOk;
}

const char* dllm_hip_trainer_tensor_name(dllm_hip_trainer* t, int64_t i) {
    const int64_t n = t ? static_cast<int64_t>(t->tensors.size()) : 0;
    if (!t || i < 0 || i >= n + static_cast<int64_t>(t->adapters.size())) return nullptr;
    return i < n ? t->tensors[static_cast<size_t>(i)].name.c_str() : t->adapters[static_cast<size_t>(i - n)].name.c_str();
}

int dllm_hip_trainer_gradients(dllm_hip_trainer* t, const int64_t* tokens, const int64_t* offsets,
                               const int64_t* lengths, int64_t windows, double scale, double router_scale,
                               double* loss, void* stream) {
    DLLM_REQUIRE(t && tokens && offsets && lengths, "null argument");
    return t->gradients(tokens, offsets, lengths, windows, scale, router_scale, loss, nullptr,
                        static_cast<hipStream_t>(stream));
}

int dllm_hip_trainer_router_loss(dllm_hip_trainer* t, double* router_loss) {
    DLLM_REQUIRE(t && router_loss, "null argument");
    *router_loss = t->last_router_loss;
    return kOk;
}

int dllm_hip_trainer_step(dllm_hip_trainer* t, const int64_t* tokens, const int64_t* offsets, const int64_t* lengths,
                          int64_t windows, const dllm_hip_adamw* adamw, double* loss, double* grad_norm,
                          void* stream) {
    DLLM_REQUIRE(t && tokens && offsets && lengths && adamw, "null argument");
    return t->step(tokens, offsets, lengths, windows, adamw, loss, grad_norm, static_cast<hipStream_t>(stream));
}

int dllm_hip_trainer_dpo_step(dllm_hip_trainer* t, const int64_t* tokens, const int64_t* offsets,
                              const int64_t* lengths, const int64_t* prompt_lengths, int64_t pairs,
                              const double* reference, double beta, const dllm_hip_adamw* adamw, double* loss,
                              double* grad_norm, void* stream) {
    DLLM_REQUIRE(t && tokens && offsets && lengths && prompt_lengths && reference && adamw, "null argument");
    return t->dpo_step(tokens, offsets, lengths, prompt_lengths, pairs, reference, beta, adamw, loss, grad_norm,
                       static_cast<hipStream_t>(stream));
}

int dllm_hip_trainer_log_probabilities(dllm_hip_trainer* t, const int64_t* tokens, const int64_t* offsets,
                                       const int64_t* lengths, const int64_t* prompt_lengths, int64_t windows,
                                       double* out, void* stream) {
    DLLM_REQUIRE(t && tokens && offsets && lengths && prompt_lengths && out, "null argument");
    return t->log_probabilities(tokens, offsets, lengths, prompt_lengths, windows, out,
                                static_cast<hipStream_t>(stream));
}

int dllm_hip_trainer_fingerprint(dllm_hip_trainer* t, int kind, char* hex_out, void* stream) {
    DLLM_REQUIRE(t && hex_out, "null argument");
    DLLM_REQUIRE(kind == kModelFile || kind == kCheckpointFile, "kind must be 0 (model.dllm) or 1 (.dllmckpt)");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<TensorSource> src;
    DLLM_TRY(t->file_tensors(kind, &src, s));
    return stream_tensor_data(src.data(), src.size(), nullptr, hex_out, s);
}

int dllm_hip_trainer_write_file(dllm_hip_trainer* t, int kind, const char* path, const char* header,
                                size_t header_len, char* hex_out, void* stream) {
    DLLM_REQUIRE(t && path && header && hex_out, "null argument");
    DLLM_REQUIRE(kind == kModelFile || kind == kCheckpointFile, "kind must be 0 (model.dllm) or 1 (.dllmckpt)");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<TensorSource> src;
    DLLM_TRY(t->file_tensors(kind, &src, s));
    return write_tensor_file(path, kind, header, header_len, src.data(), src.size(), hex_out, s);
}

int dllm_hip_trainer_read_checkpoint(dllm_hip_trainer* t, const char* path, const char* fingerprint, void* stream) {
    DLLM_REQUIRE(t && path && fingerprint, "null argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    std::vector<TensorSource> src;
    DLLM_TRY(t->file_tensors(kCheckpointFile, &src, s));
    char hex[65];
    // verify the whole data section first (trainer.py:593-594), then load it
    DLLM_TRY(read_tensor_file_data(path, kCheckpointFile, nullptr, 0, hex, 0, s));
    DLLM_REQUIRE(strncmp(hex, fingerprint, 64) == 0 && strlen(fingerprint) == 64,
                 std::string(path) + ": tensor data does not match the fingerprint (corrupt file?)");
    DLLM_TRY(read_tensor_file_data(path, kCheckpointFile, src.data(), src.size(), hex, 1, s));
    DLLM_REQUIRE(strncmp(hex, fingerprint, 64) == 0, std::string(path) + ": the file changed while it was read");
    t->wt_valid = false;  // new parameters: transposes, merged weights and the quantised base are rebuilt
    t->merged_valid = false;
    if (t->lora_on && t->lc.base_quantize) t->base_ready = false;
    return kOk;
}

}  // extern "C"
