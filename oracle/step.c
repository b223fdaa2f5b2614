/*
 * CPU oracle of the training step orchestration (TEST INFRASTRUCTURE ONLY; see oracle.h).
 *
 * Restates, per window, DecoderGradients (src/etalii_dllm/training/backprop.py:88-118, 183-357, 359-377, 399-527),
 * and per step FineTuner._language_model_gradients (training/trainer.py:312-335) and AdamW.step
 * (training/optimizer.py:59-109), calling kernels through an orc_ops table. The float32 glue between kernel calls
 * (NumPy in the reference) is written as single float operations in the reference's operand order.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

int64_t orc_layer_slots(const orc_config* c) { return ORC_LAYER_FIXED + 3 * c->experts; }
int64_t orc_slot_count(const orc_config* c) { return ORC_GLOBALS + c->layers * orc_layer_slots(c); }
int64_t orc_slot(const orc_config* c, int64_t layer, int64_t kind) {
    return ORC_GLOBALS + layer * orc_layer_slots(c) + kind;
}
int64_t orc_expert_slot(const orc_config* c, int64_t layer, int64_t expert, int64_t which) {
    return orc_slot(c, layer, ORC_LAYER_FIXED + 3 * expert + which);
}

static int has_pre_norms(const orc_config* c) { return c->norm_placement != 1; }
static int has_post_norms(const orc_config* c) { return c->norm_placement != 0; }

int orc_is_sparse(const orc_config* c, int64_t layer) {
    if (c->experts <= 0) return 0;
    if (c->dense_layer_flags) return !c->dense_layer_flags[layer];
    return !(layer < 64 && ((c->dense_layers >> layer) & 1));
}

/* Shapes of architecture.py:418-468 for the decoder families a step here covers. */
static int64_t slot_shape(const orc_config* c, int64_t slot, int64_t* d0, int64_t* d1) {
    const int64_t H = c->hidden, q = c->heads * c->head_dim, kv = c->kv_heads * c->head_dim;
    *d1 = 0;
    if (slot == ORC_EMBEDDING) { *d0 = c->vocab; *d1 = H; return 2; }
    if (slot == ORC_FINAL_NORM) { *d0 = H; return 1; }
    if (slot == ORC_LM_HEAD) { if (c->tied) return 0; *d0 = c->vocab; *d1 = H; return 2; }
    const int64_t kind = (slot - ORC_GLOBALS) % orc_layer_slots(c);
    const int sparse = orc_is_sparse(c, (slot - ORC_GLOBALS) / orc_layer_slots(c));
    switch (kind) {
        case ORC_ATTN_NORM: case ORC_MLP_NORM: if (!has_pre_norms(c)) return 0; *d0 = H; return 1;
        case ORC_ATTN_POST_NORM: case ORC_MLP_POST_NORM: if (!has_post_norms(c)) return 0; *d0 = H; return 1;
        case ORC_Q: *d0 = q; *d1 = H; return 2;
        case ORC_K: case ORC_V: *d0 = kv; *d1 = H; return 2;
        case ORC_QB: if (!c->attn_bias) return 0; *d0 = q; return 1;
        case ORC_KB: case ORC_VB: if (!c->attn_bias) return 0; *d0 = kv; return 1;
        case ORC_QNORM: if (!c->qk_norm) return 0; *d0 = c->qk_norm == 2 ? q : c->head_dim; return 1;
        case ORC_KNORM: if (!c->qk_norm) return 0; *d0 = c->qk_norm == 2 ? kv : c->head_dim; return 1;
        case ORC_O: *d0 = H; *d1 = q; return 2;
        case ORC_GATE: case ORC_UP: if (sparse) return 0; *d0 = c->inter; *d1 = H; return 2;
        case ORC_DOWN: if (sparse) return 0; *d0 = H; *d1 = c->inter; return 2;
        case ORC_ROUTER: if (!sparse) return 0; *d0 = c->experts; *d1 = H; return 2;
        case ORC_SHARED_GATE: case ORC_SHARED_UP:
            if (!sparse || c->shared_inter == 0) return 0;
            *d0 = c->shared_inter; *d1 = H; return 2;
        case ORC_SHARED_DOWN: if (!sparse || c->shared_inter == 0) return 0; *d0 = H; *d1 = c->shared_inter; return 2;
        case ORC_SHARED_GATE_W: if (!sparse || c->shared_inter == 0 || !c->shared_gate) return 0; *d0 = 1; *d1 = H; return 2;
        default: {
            if (!sparse) return 0;
            const int64_t which = (kind - ORC_LAYER_FIXED) % 3;
            if (which == 2) { *d0 = H; *d1 = c->expert_inter; } else { *d0 = c->expert_inter; *d1 = H; }
            return 2;
        }
    }
}

int64_t orc_tensor_numel(const orc_config* c, int64_t slot) {
    int64_t d0 = 0, d1 = 0;
    const int64_t nd = slot_shape(c, slot, &d0, &d1);
    if (nd == 0) return 0;
    return nd == 1 ? d0 : d0 * d1;
}

int orc_tensor_ndim(const orc_config* c, int64_t slot) {
    int64_t d0, d1;
    return (int)slot_shape(c, slot, &d0, &d1);
}

static float* falloc(int64_t n) { return (float*)calloc((size_t)(n > 0 ? n : 1), sizeof(float)); }

/* Elementwise float32 glue: out = a + b, out = a * b (one IEEE float operation per element). */
static void vadd(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] + b[i];
}
static void vmul(const float* a, const float* b, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = a[i] * b[i];
}

/* The saved activations of one dense SwiGLU block or one expert group (backprop.py:492-499). */
typedef struct {
    int64_t rows;
    int64_t* row_index; /* expert groups: the rows routed to this expert, ascending */
    int64_t* rank;      /* and the rank of this expert in each row's choice */
    float *x, *gate, *up, *gate_act, *product, *y;
} swiglu_saved;

typedef struct {
    float *x_in, *h1, *q_raw, *k_raw, *q, *k, *v, *attended, *out, *x_mid, *h2, *mlp;
    float *out_normed, *mlp_normed; /* post norms: the normalised block outputs (NULL without) */
    swiglu_saved dense;
    swiglu_saved shared; /* the shared expert over every row (rows == 0 without one) */
    float* shared_s;     /* [n]: its gate's sigmoid */
    float* router_logits; /* [n, experts] */
    int64_t* chosen;      /* [n, topk] */
    float* routing;       /* [n, topk] */
    swiglu_saved* groups; /* [experts]; rows == 0 when no row chose the expert */
} layer_saved;

static void swiglu_forward(const orc_ops* ops, float* const* w, int64_t gate_slot, int64_t up_slot, int64_t down_slot,
                           int64_t inter, int64_t H, swiglu_saved* s, int act) {
    const int64_t n = s->rows;
    s->gate = falloc(n * inter);
    s->up = falloc(n * inter);
    s->gate_act = falloc(n * inter);
    s->product = falloc(n * inter);
    s->y = falloc(n * H);
    ops->linear(s->x, w[gate_slot], NULL, s->gate, n, H, inter);
    ops->linear(s->x, w[up_slot], NULL, s->up, n, H, inter);
    if (act == 1)
        ops->gelu_tanh(s->gate, s->gate_act, n * inter);
    else
        ops->silu(s->gate, s->gate_act, n * inter);
    vmul(s->gate_act, s->up, s->product, n * inter);
    ops->linear(s->product, w[down_slot], NULL, s->y, n, inter, H);
}

static void swiglu_free(swiglu_saved* s) {
    free(s->gate); free(s->up); free(s->gate_act); free(s->product); free(s->y);
}

/* _swiglu_backward (backprop.py:289-306): returns dx = dx_gate + dx_up in `dx`. */
static void swiglu_backward(const orc_ops* ops, float* const* w, float* const* g, int64_t gate_slot, int64_t up_slot,
                            int64_t down_slot, int64_t inter, int64_t H, const swiglu_saved* s, const float* dy,
                            float* dx, int act) {
    const int64_t n = s->rows;
    float* dproduct = falloc(n * inter);
    float* t = falloc(n * inter);
    float* dgate = falloc(n * inter);
    float* dup = falloc(n * inter);
    float* dx_gate = falloc(n * H);
    float* dx_up = falloc(n * H);
    ops->linear_backward(s->product, w[down_slot], dy, dproduct, g[down_slot], NULL, n, inter, H);
    vmul(dproduct, s->up, t, n * inter);
    if (act == 1)
        ops->gelu_tanh_backward(s->gate, t, dgate, n * inter);
    else
        ops->silu_backward(s->gate, t, dgate, n * inter);
    vmul(dproduct, s->gate_act, dup, n * inter);
    ops->linear_backward(s->x, w[gate_slot], dgate, dx_gate, g[gate_slot], NULL, n, H, inter);
    ops->linear_backward(s->x, w[up_slot], dup, dx_up, g[up_slot], NULL, n, H, inter);
    vadd(dx_gate, dx_up, dx, n * H);
    free(dproduct); free(t); free(dgate); free(dup); free(dx_gate); free(dx_up);
}

typedef struct {
    const orc_ops* ops;
    const orc_config* c;
    float* const* w;
    int64_t n;
    int64_t* positions;
    double* inv_freq;
    double* local_inv_freq; /* the windowed layers' (Gemma 3), or inv_freq itself */
    layer_saved* layers;
    float* final_input;
    float* hidden;
} fwd_state;

/* TransformerConfig.window (architecture.py:353-359): the layer's window, 0 for full causal attention. */
static int64_t layer_window(const orc_config* c, int64_t layer) {
    if (c->window == 0) return 0;
    if (c->full_attention_layer_flags) return c->full_attention_layer_flags[layer] ? 0 : c->window;
    return layer < 64 && ((c->full_attention_layers >> layer) & 1) ? 0 : c->window;
}

/* The inverse frequencies layer l rotates with (uses_local_rope, architecture.py:322-324). */
static const double* layer_inv_freq(const fwd_state* st, int64_t layer) {
    return st->c->local_rope_theta != 0.0 && layer_window(st->c, layer) != 0 ? st->local_inv_freq : st->inv_freq;
}

/* A multiplier of the config that is present (neither 1 nor unset). */
static int has_multiplier(double m) { return m != 0.0 && m != 1.0; }

/* x = x * f, elementwise in float (numpy's array times np.float32). */
static void vscale(float* x, float f, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] * f;
}

/* x = x / f, elementwise in float (_finish, backprop.py:174-181, and the head gradient, :197-200). */
static void vdivide(float* x, float f, int64_t n) {
    for (int64_t i = 0; i < n; ++i) x[i] = x[i] / f;
}

/* _forward (backprop.py:399-490) and _experts (backprop.py:501-527). */
static void forward(fwd_state* st, const int64_t* tokens) {
    const orc_ops* ops = st->ops;
    const orc_config* c = st->c;
    float* const* w = st->w;
    const int64_t n = st->n, H = c->hidden, hd = c->head_dim;
    const int64_t qd = c->heads * hd, kvd = c->kv_heads * hd;
    float* x = falloc(n * H);
    for (int64_t t = 0; t < n; ++t) memcpy(x + t * H, w[ORC_EMBEDDING] + tokens[t] * H, (size_t)H * sizeof(float));
    if (has_multiplier(c->embedding_multiplier)) vscale(x, (float)c->embedding_multiplier, n * H);
    for (int64_t l = 0; l < c->layers; ++l) {
        layer_saved* s = &st->layers[l];
        memset(s, 0, sizeof *s);
        s->x_in = x;
        s->h1 = falloc(n * H);
        if (has_pre_norms(c))
            ops->rms_norm(x, w[orc_slot(c, l, ORC_ATTN_NORM)], s->h1, n, H, c->eps, (int)c->norm_unit_offset);
        else
            memcpy(s->h1, x, (size_t)(n * H) * sizeof(float));
        s->q_raw = falloc(n * qd);
        s->k_raw = falloc(n * kvd);
        s->v = falloc(n * kvd);
        ops->linear(s->h1, w[orc_slot(c, l, ORC_Q)], w[orc_slot(c, l, ORC_QB)], s->q_raw, n, H, qd);
        ops->linear(s->h1, w[orc_slot(c, l, ORC_K)], w[orc_slot(c, l, ORC_KB)], s->k_raw, n, H, kvd);
        ops->linear(s->h1, w[orc_slot(c, l, ORC_V)], w[orc_slot(c, l, ORC_VB)], s->v, n, H, kvd);
        const float* qn = s->q_raw;
        const float* kn = s->k_raw;
        float* qtmp = NULL;
        float* ktmp = NULL;
        if (c->qk_norm) {
            qtmp = falloc(n * qd);
            ktmp = falloc(n * kvd);
            if (c->qk_norm == 2) {
                ops->rms_norm(s->q_raw, w[orc_slot(c, l, ORC_QNORM)], qtmp, n, qd, c->eps, (int)c->norm_unit_offset);
                ops->rms_norm(s->k_raw, w[orc_slot(c, l, ORC_KNORM)], ktmp, n, kvd, c->eps, (int)c->norm_unit_offset);
            } else {
                ops->rms_norm(s->q_raw, w[orc_slot(c, l, ORC_QNORM)], qtmp, n * c->heads, hd, c->eps, (int)c->norm_unit_offset);
                ops->rms_norm(s->k_raw, w[orc_slot(c, l, ORC_KNORM)], ktmp, n * c->kv_heads, hd, c->eps, (int)c->norm_unit_offset);
            }
            qn = qtmp;
            kn = ktmp;
        }
        s->q = falloc(n * qd);
        s->k = falloc(n * kvd);
        ops->rope(qn, st->positions, layer_inv_freq(st, l), s->q, n, c->heads, hd, c->rotary_dim, 0, 0);
        ops->rope(kn, st->positions, layer_inv_freq(st, l), s->k, n, c->kv_heads, hd, c->rotary_dim, 0, 0);
        free(qtmp);
        free(ktmp);
        s->attended = falloc(n * qd);
        ops->attention(s->q, s->k, s->v, s->attended, n, n, c->heads, c->kv_heads, hd, hd, c->attention_scale, 1, 0,
                       layer_window(c, l), c->attention_softcap);
        s->out = falloc(n * H);
        ops->linear(s->attended, w[orc_slot(c, l, ORC_O)], NULL, s->out, n, qd, H);
        s->x_mid = falloc(n * H);
        if (has_post_norms(c)) {
            s->out_normed = falloc(n * H);
            ops->rms_norm(s->out, w[orc_slot(c, l, ORC_ATTN_POST_NORM)], s->out_normed, n, H, c->eps, (int)c->norm_unit_offset);
        }
        vadd(x, has_post_norms(c) ? s->out_normed : s->out, s->x_mid, n * H);
        s->h2 = falloc(n * H);
        if (has_pre_norms(c))
            ops->rms_norm(s->x_mid, w[orc_slot(c, l, ORC_MLP_NORM)], s->h2, n, H, c->eps, (int)c->norm_unit_offset);
        else
            memcpy(s->h2, s->x_mid, (size_t)(n * H) * sizeof(float));
        if (!orc_is_sparse(c, l)) {
            s->dense.rows = n;
            s->dense.x = s->h2;
            swiglu_forward(ops, w, orc_slot(c, l, ORC_GATE), orc_slot(c, l, ORC_UP), orc_slot(c, l, ORC_DOWN), c->inter,
                           H, &s->dense, (int)c->activation);
            s->mlp = s->dense.y;
        } else {
            const int64_t E = c->experts, K = c->topk;
            s->router_logits = falloc(n * E);
            ops->linear(s->h2, w[orc_slot(c, l, ORC_ROUTER)], NULL, s->router_logits, n, H, E);
            s->chosen = (int64_t*)calloc((size_t)(n * K), sizeof(int64_t));
            s->routing = falloc(n * K);
            ops->moe_route(s->router_logits, s->chosen, s->routing, n, E, K, (int)c->normalize);
            s->mlp = falloc(n * H); /* zeros */
            s->groups = (swiglu_saved*)calloc((size_t)E, sizeof(swiglu_saved));
            for (int64_t e = 0; e < E; ++e) {
                swiglu_saved* gsv = &s->groups[e];
                int64_t count = 0;
                for (int64_t i = 0; i < n * K; ++i) count += s->chosen[i] == e;
                if (count == 0) continue;
                gsv->rows = count;
                gsv->row_index = (int64_t*)malloc((size_t)count * sizeof(int64_t));
                gsv->rank = (int64_t*)malloc((size_t)count * sizeof(int64_t));
                gsv->x = falloc(count * H);
                int64_t m = 0;
                for (int64_t r = 0; r < n; ++r)
                    for (int64_t j = 0; j < K; ++j)
                        if (s->chosen[r * K + j] == e) {
                            gsv->row_index[m] = r;
                            gsv->rank[m] = j;
                            memcpy(gsv->x + m * H, s->h2 + r * H, (size_t)H * sizeof(float));
                            ++m;
                        }
                swiglu_forward(ops, w, orc_expert_slot(c, l, e, 0), orc_expert_slot(c, l, e, 1),
                               orc_expert_slot(c, l, e, 2), c->expert_inter, H, gsv, (int)c->activation);
                for (int64_t i = 0; i < count; ++i) {
                    const float weight = s->routing[gsv->row_index[i] * K + gsv->rank[i]];
                    float* o = s->mlp + gsv->row_index[i] * H;
                    for (int64_t d = 0; d < H; ++d) o[d] = o[d] + gsv->y[i * H + d] * weight;
                }
            }
            if (c->shared_inter > 0) { /* out = out + y (times the gate's sigmoid) */
                s->shared.rows = n;
                s->shared.x = s->h2;
                swiglu_forward(ops, w, orc_slot(c, l, ORC_SHARED_GATE), orc_slot(c, l, ORC_SHARED_UP),
                               orc_slot(c, l, ORC_SHARED_DOWN), c->shared_inter, H, &s->shared, (int)c->activation);
                if (c->shared_gate) {
                    s->shared_s = falloc(n);
                    ops->linear(s->h2, w[orc_slot(c, l, ORC_SHARED_GATE_W)], NULL, s->shared_s, n, H, 1);
                    for (int64_t r = 0; r < n; ++r) s->shared_s[r] = (float)orc_sigmoid((double)s->shared_s[r]);
                }
                for (int64_t r = 0; r < n; ++r)
                    for (int64_t d = 0; d < H; ++d) {
                        const float y = s->shared.y[r * H + d];
                        s->mlp[r * H + d] = s->mlp[r * H + d] + (c->shared_gate ? y * s->shared_s[r] : y);
                    }
            }
        }
        float* x_out = falloc(n * H);
        if (has_post_norms(c)) {
            s->mlp_normed = falloc(n * H);
            ops->rms_norm(s->mlp, w[orc_slot(c, l, ORC_MLP_POST_NORM)], s->mlp_normed, n, H, c->eps, (int)c->norm_unit_offset);
        }
        vadd(s->x_mid, has_post_norms(c) ? s->mlp_normed : s->mlp, x_out, n * H);
        x = x_out;
    }
    st->final_input = x;
    st->hidden = falloc(n * H);
    ops->rms_norm(x, w[ORC_FINAL_NORM], st->hidden, n, H, c->eps, (int)c->norm_unit_offset);
}

static void free_state(fwd_state* st) {
    const orc_config* c = st->c;
    for (int64_t l = 0; l < c->layers; ++l) {
        layer_saved* s = &st->layers[l];
        free(s->x_in); free(s->h1); free(s->q_raw); free(s->k_raw); free(s->q); free(s->k); free(s->v);
        free(s->attended); free(s->out); free(s->x_mid); free(s->h2); free(s->out_normed); free(s->mlp_normed);
        if (!orc_is_sparse(c, l)) {
            swiglu_free(&s->dense);
        } else {
            free(s->mlp); free(s->router_logits); free(s->chosen); free(s->routing);
            for (int64_t e = 0; e < c->experts; ++e) {
                swiglu_saved* g = &s->groups[e];
                if (g->rows == 0) continue;
                free(g->row_index); free(g->rank); free(g->x);
                swiglu_free(g);
            }
            free(s->groups);
            if (s->shared.rows) swiglu_free(&s->shared);
            free(s->shared_s);
        }
    }
    free(st->final_input);
    free(st->hidden);
    free(st->layers);
    free(st->positions);
    if (st->local_inv_freq != st->inv_freq) free(st->local_inv_freq);
    free(st->inv_freq);
}

static void init_state(fwd_state* st, const orc_ops* ops, const orc_config* c, float* const* w, int64_t n) {
    st->ops = ops;
    st->c = c;
    st->w = w;
    st->n = n;
    st->positions = (int64_t*)malloc((size_t)n * sizeof(int64_t));
    for (int64_t t = 0; t < n; ++t) st->positions[t] = t;
    st->inv_freq = (double*)malloc((size_t)(c->rotary_dim / 2 + 1) * sizeof(double));
    if (c->inv_freq)
        memcpy(st->inv_freq, c->inv_freq, (size_t)(c->rotary_dim / 2) * sizeof(double));
    else
        orc_rope_inv_freq((size_t)c->rotary_dim, c->rope_theta, st->inv_freq);
    st->local_inv_freq = st->inv_freq;
    if (c->local_rope_theta != 0.0) {
        st->local_inv_freq = (double*)malloc((size_t)(c->rotary_dim / 2 + 1) * sizeof(double));
        orc_rope_inv_freq((size_t)c->rotary_dim, c->local_rope_theta, st->local_inv_freq);
    }
    st->layers = (layer_saved*)calloc((size_t)c->layers, sizeof(layer_saved));
}

/* rope_scaled_tensors (transformer.py:204-209): the QK-norm weights when the model has QK-norm, else the q and k
 * projections and their biases. */
static int rope_scaled_slots(const orc_config* c, int64_t layer, int64_t* out) {
    int k = 0;
    if (c->qk_norm) {
        out[k++] = orc_slot(c, layer, ORC_QNORM);
        out[k++] = orc_slot(c, layer, ORC_KNORM);
    } else {
        out[k++] = orc_slot(c, layer, ORC_Q);
        out[k++] = orc_slot(c, layer, ORC_K);
        if (c->attn_bias) {
            out[k++] = orc_slot(c, layer, ORC_QB);
            out[k++] = orc_slot(c, layer, ORC_KB);
        }
    }
    return k;
}

/* _rope_scaled (transformer.py:212-221) and _unfold (backprop.py:388-393): the entries of each head's first
 * rotary_dim rows times f32(factor), elementwise in float. */
static void scale_rotary_rows(const orc_config* c, int64_t slot, const float* src, float* dst, float factor) {
    int64_t d0 = 0, d1 = 0;
    const int nd = (int)slot_shape(c, slot, &d0, &d1);
    const int64_t cols = nd == 2 ? d1 : 1;
    for (int64_t r = 0; r < d0; ++r) {
        const int rotated = (r % c->head_dim) < c->rotary_dim;
        for (int64_t j = 0; j < cols; ++j) dst[r * cols + j] = rotated ? src[r * cols + j] * factor : src[r * cols + j];
    }
}

/* The tensors the residual multiplier folds into (fold_scales, transformer.py:231-239): every name ending in
 * "attention.o.weight" or "down.weight", so each layer's output projection and its MLP's (or every expert's) down
 * projection. */
static int residual_scaled_slots(const orc_config* c, int64_t layer, int64_t* out) {
    int k = 0;
    out[k++] = orc_slot(c, layer, ORC_O);
    if (!orc_is_sparse(c, layer)) {
        out[k++] = orc_slot(c, layer, ORC_DOWN);
    } else {
        for (int64_t e = 0; e < c->experts; ++e) out[k++] = orc_expert_slot(c, layer, e, 2);
        if (c->shared_inter > 0) out[k++] = orc_slot(c, layer, ORC_SHARED_DOWN);
    }
    return k;
}

/* fold_scales (transformer.py:224-245) over a weight table: a table whose residual-scaled and rope-scaled slots point
 * to folded copies (owned[] holds them, to free), or NULL when neither the residual multiplier nor the RoPE attention
 * factor is present. The two sets of tensors are disjoint. */
static float** fold_weights(const orc_config* c, float* const* w, float*** owned_out) {
    const double a = c->rope_attention_factor;
    const int rope = has_multiplier(a), residual = has_multiplier(c->residual_multiplier);
    *owned_out = NULL;
    if (!rope && !residual) return NULL;
    const int64_t slots = orc_slot_count(c);
    float** folded = (float**)calloc((size_t)slots, sizeof(float*));
    float** owned = (float**)calloc((size_t)slots, sizeof(float*));
    for (int64_t s = 0; s < slots; ++s) folded[s] = w[s];
    int64_t* list = (int64_t*)malloc((size_t)(c->experts + 5) * sizeof(int64_t));
    for (int64_t l = 0; l < c->layers; ++l) {
        if (residual) {
            const int k = residual_scaled_slots(c, l, list);
            for (int i = 0; i < k; ++i) {
                const int64_t numel = orc_tensor_numel(c, list[i]);
                owned[list[i]] = falloc(numel);
                memcpy(owned[list[i]], w[list[i]], (size_t)numel * sizeof(float));
                vscale(owned[list[i]], (float)c->residual_multiplier, numel);
                folded[list[i]] = owned[list[i]];
            }
        }
        if (rope) {
            const int k = rope_scaled_slots(c, l, list);
            for (int i = 0; i < k; ++i) {
                owned[list[i]] = falloc(orc_tensor_numel(c, list[i]));
                scale_rotary_rows(c, list[i], w[list[i]], owned[list[i]], (float)a);
                folded[list[i]] = owned[list[i]];
            }
        }
    }
    free(list);
    *owned_out = owned;
    return folded;
}

static void free_folded(const orc_config* c, float** folded, float** owned) {
    if (!folded) return;
    for (int64_t s = 0; s < orc_slot_count(c); ++s) free(owned[s]);
    free(owned);
    free(folded);
}

int orc_logits(const orc_ops* ops, const orc_config* c, float* const* w_stored, const int64_t* tokens, int64_t n,
               float* logits) {
    float** owned;
    float** folded = fold_weights(c, w_stored, &owned);
    float* const* w = folded ? folded : w_stored;
    fwd_state st;
    init_state(&st, ops, c, w, n);
    forward(&st, tokens);
    ops->linear(st.hidden, w[c->tied ? ORC_EMBEDDING : ORC_LM_HEAD], NULL, logits, n, c->hidden, c->vocab);
    if (has_multiplier(c->logits_scaling)) vdivide(logits, (float)c->logits_scaling, n * c->vocab);
    if (c->logits_softcap != 0.0) ops->softcap(logits, logits, (size_t)(n * c->vocab), c->logits_softcap);
    free_state(&st);
    free_folded(c, folded, owned);
    return 0;
}

/* _router_loss (backprop.py:359-377): the loss, and the gradient row (broadcast to every row of every sparse layer). */
static double router_loss(const fwd_state* st, double router_scale, float* grad_row) {
    const orc_ops* ops = st->ops;
    const orc_config* c = st->c;
    const int64_t n = st->n, E = c->experts, K = c->topk, L = c->layers;
    int64_t sparse_layers = 0;
    for (int64_t l = 0; l < L; ++l) sparse_layers += orc_is_sparse(c, l);
    const int64_t rows = n * sparse_layers;
    float* probs = falloc(rows * E);
    int64_t* counts = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    for (int64_t l = 0, b = 0; l < L; ++l) {
        if (!orc_is_sparse(c, l)) continue;
        const layer_saved* s = &st->layers[l];
        for (int64_t r = 0; r < n; ++r) ops->softmax(s->router_logits + r * E, probs + (b * n + r) * E, E);
        for (int64_t i = 0; i < n * K; ++i) counts[s->chosen[i]] += 1;
        ++b;
    }
    float* fractions = falloc(E);
    float* means = falloc(E);
    for (int64_t e = 0; e < E; ++e) fractions[e] = (float)((double)counts[e] / (double)rows);
    ops->column_mean(probs, means, rows, E);
    const double loss = (double)E * (double)ops->dot(fractions, means, E); /* Python float product */
    if (grad_row)
        for (int64_t e = 0; e < E; ++e)
            grad_row[e] = (float)(router_scale * (double)E * (double)counts[e] / (double)(rows * rows));
    free(probs); free(counts); free(fractions); free(means);
    return loss;
}

/* _experts_backward (backprop.py:308-357) for routed experts without a shared expert. */
static void experts_backward(const fwd_state* st, int64_t l, const float* dmlp, float* const* g,
                             const float* dprob_row, float* dh2) {
    const orc_ops* ops = st->ops;
    const orc_config* c = st->c;
    float* const* w = st->w;
    const layer_saved* s = &st->layers[l];
    const int64_t n = st->n, H = c->hidden, E = c->experts, K = c->topk;
    memset(dh2, 0, (size_t)(n * H) * sizeof(float));
    float* dweights = falloc(n * K);
    for (int64_t e = 0; e < E; ++e) {
        const swiglu_saved* gsv = &s->groups[e];
        if (gsv->rows == 0) {
            for (int64_t which = 0; which < 3; ++which) {
                const int64_t slot = orc_expert_slot(c, l, e, which);
                memset(g[slot], 0, (size_t)orc_tensor_numel(c, slot) * sizeof(float));
            }
            continue;
        }
        const int64_t m = gsv->rows;
        float* dout = falloc(m * H);
        float* dy = falloc(m * H);
        float* dx = falloc(m * H);
        for (int64_t i = 0; i < m; ++i) {
            const int64_t row = gsv->row_index[i];
            memcpy(dout + i * H, dmlp + row * H, (size_t)H * sizeof(float));
            dweights[row * K + gsv->rank[i]] = ops->dot(dout + i * H, gsv->y + i * H, H);
            const float weight = s->routing[row * K + gsv->rank[i]];
            for (int64_t d = 0; d < H; ++d) dy[i * H + d] = dout[i * H + d] * weight;
        }
        swiglu_backward(ops, w, g, orc_expert_slot(c, l, e, 0), orc_expert_slot(c, l, e, 1),
                        orc_expert_slot(c, l, e, 2), c->expert_inter, H, gsv, dy, dx, (int)c->activation);
        for (int64_t i = 0; i < m; ++i) {
            float* o = dh2 + gsv->row_index[i] * H;
            for (int64_t d = 0; d < H; ++d) o[d] = o[d] + dx[i * H + d];
        }
        free(dout); free(dy); free(dx);
    }
    float* dprob = NULL;
    if (dprob_row) {
        dprob = falloc(n * E);
        for (int64_t r = 0; r < n; ++r) memcpy(dprob + r * E, dprob_row, (size_t)E * sizeof(float));
    }
    if (c->shared_inter > 0) { /* the shared expert and its gate (backprop.py:339-351) */
        float* dy = falloc(n * H);
        float* dscore = falloc(n);
        float* dxs = falloc(n * H);
        for (int64_t r = 0; r < n; ++r) {
            if (c->shared_gate) {
                const float sg = s->shared_s[r];
                for (int64_t d = 0; d < H; ++d) dy[r * H + d] = dmlp[r * H + d] * sg;
                const float ds = ops->dot(dmlp + r * H, s->shared.y + r * H, H);
                dscore[r] = (ds * sg) * (1.0f - sg);
            } else {
                memcpy(dy + r * H, dmlp + r * H, (size_t)H * sizeof(float));
            }
        }
        swiglu_backward(ops, w, g, orc_slot(c, l, ORC_SHARED_GATE), orc_slot(c, l, ORC_SHARED_UP),
                        orc_slot(c, l, ORC_SHARED_DOWN), c->shared_inter, H, &s->shared, dy, dxs, (int)c->activation);
        vadd(dh2, dxs, dh2, n * H);
        if (c->shared_gate) {
            const int64_t gs = orc_slot(c, l, ORC_SHARED_GATE_W);
            ops->linear_backward(s->h2, w[gs], dscore, dxs, g[gs], NULL, n, H, 1);
            vadd(dh2, dxs, dh2, n * H);
        }
        free(dy); free(dscore); free(dxs);
    }
    float* dlogits = falloc(n * E);
    ops->moe_route_backward(s->router_logits, s->chosen, dweights, dprob, dlogits, n, E, K, (int)c->normalize);
    float* dh2_router = falloc(n * H);
    const int64_t rs = orc_slot(c, l, ORC_ROUTER);
    ops->linear_backward(s->h2, w[rs], dlogits, dh2_router, g[rs], NULL, n, H, E);
    vadd(dh2, dh2_router, dh2, n * H);
    free(dweights); free(dprob); free(dlogits); free(dh2_router);
}

static int window_gradients(const orc_ops* ops, const orc_config* c, float* const* w, const int64_t* tokens,
                            const int64_t* targets, int64_t n, double scale, double router_scale, float* const* g,
                            double* loss, double* router_loss_out) {
    if (n <= 0) return -1;
    for (int64_t t = 0; t < n; ++t)
        if (tokens[t] < 0 || tokens[t] >= c->vocab) return -2;
    fwd_state st;
    init_state(&st, ops, c, w, n);
    forward(&st, tokens);
    const int64_t H = c->hidden, V = c->vocab, hd = c->head_dim;
    const int64_t qd = c->heads * hd, kvd = c->kv_heads * hd;

    float* grad_row = NULL;
    double rl = 0.0;
    if (c->experts > 0) {
        grad_row = falloc(c->experts);
        rl = router_loss(&st, router_scale, grad_row);
    }
    if (router_loss_out) *router_loss_out = rl;

    /* _backward_from_logits (backprop.py:183-206) */
    const float* head = w[c->tied ? ORC_EMBEDDING : ORC_LM_HEAD];
    float* logits = falloc(n * V);
    float* dlogits = falloc(n * V);
    ops->linear(st.hidden, head, NULL, logits, n, H, V);
    if (has_multiplier(c->logits_scaling)) vdivide(logits, (float)c->logits_scaling, n * V);
    float* capped = NULL; /* _finish (backprop.py:174-181): the capped logits; `logits` keeps the uncapped ones */
    if (c->logits_softcap != 0.0) {
        capped = falloc(n * V);
        ops->softcap(logits, capped, (size_t)(n * V), c->logits_softcap);
    }
    *loss = ops->cross_entropy(capped ? capped : logits, targets, dlogits, n, V, scale);
    if (capped) ops->softcap_backward(logits, dlogits, dlogits, (size_t)(n * V), c->logits_softcap);
    free(capped);
    free(logits);
    if (has_multiplier(c->logits_scaling)) vdivide(dlogits, (float)c->logits_scaling, n * V);
    float* dhidden = falloc(n * H);
    float* dhead = falloc(V * H);
    ops->linear_backward(st.hidden, head, dlogits, dhidden, dhead, NULL, n, H, V);
    free(dlogits);
    float* dx = falloc(n * H);
    ops->rms_norm_backward(st.final_input, w[ORC_FINAL_NORM], dhidden, dx, g[ORC_FINAL_NORM], n, H, c->eps, (int)c->norm_unit_offset);
    free(dhidden);

    /* _backward_layer (backprop.py:208-287), layers in reverse */
    float* dh2 = falloc(n * H);
    float* dtmp = falloc(n * H);
    float* dpost = falloc(n * H);
    float* dx_mid = falloc(n * H);
    float* dattended = falloc(n * qd);
    float* dq_t = falloc(n * qd);
    float* dk_t = falloc(n * kvd);
    float* dv_t = falloc(n * kvd);
    float* dq = falloc(n * qd);
    float* dk = falloc(n * kvd);
    float* dq2 = falloc(n * qd);
    float* dk2 = falloc(n * kvd);
    float* dh1 = falloc(n * H);
    float* dh = falloc(n * H);
    for (int64_t l = c->layers - 1; l >= 0; --l) {
        const layer_saved* s = &st.layers[l];
        const float* dmlp = dx;
        if (has_post_norms(c)) {
            const int64_t pn = orc_slot(c, l, ORC_MLP_POST_NORM);
            ops->rms_norm_backward(s->mlp, w[pn], dx, dpost, g[pn], n, H, c->eps, (int)c->norm_unit_offset);
            dmlp = dpost;
        }
        if (!orc_is_sparse(c, l)) {
            swiglu_backward(ops, w, g, orc_slot(c, l, ORC_GATE), orc_slot(c, l, ORC_UP), orc_slot(c, l, ORC_DOWN),
                            c->inter, H, &s->dense, dmlp, dh2, (int)c->activation);
        } else {
            experts_backward(&st, l, dmlp, g, router_scale != 0.0 ? grad_row : NULL, dh2);
        }
        if (has_pre_norms(c)) {
            const int64_t mn = orc_slot(c, l, ORC_MLP_NORM);
            ops->rms_norm_backward(s->x_mid, w[mn], dh2, dtmp, g[mn], n, H, c->eps, (int)c->norm_unit_offset);
            vadd(dx, dtmp, dx_mid, n * H);
        } else {
            vadd(dx, dh2, dx_mid, n * H);
        }
        const float* dout = dx_mid;
        if (has_post_norms(c)) {
            const int64_t pn = orc_slot(c, l, ORC_ATTN_POST_NORM);
            ops->rms_norm_backward(s->out, w[pn], dx_mid, dpost, g[pn], n, H, c->eps, (int)c->norm_unit_offset);
            dout = dpost;
        }
        const int64_t os = orc_slot(c, l, ORC_O);
        ops->linear_backward(s->attended, w[os], dout, dattended, g[os], NULL, n, qd, H);
        ops->attention_backward(s->q, s->k, s->v, dattended, dq_t, dk_t, dv_t, n, n, c->heads, c->kv_heads, hd, hd,
                                c->attention_scale, 1, 0, layer_window(c, l), c->attention_softcap);
        ops->rope(dq_t, st.positions, layer_inv_freq(&st, l), dq, n, c->heads, hd, c->rotary_dim, 0, 1);
        ops->rope(dk_t, st.positions, layer_inv_freq(&st, l), dk, n, c->kv_heads, hd, c->rotary_dim, 0, 1);
        const float* dqf = dq;
        const float* dkf = dk;
        if (c->qk_norm) {
            const int64_t qs = orc_slot(c, l, ORC_QNORM), ks = orc_slot(c, l, ORC_KNORM);
            if (c->qk_norm == 1) {
                ops->rms_norm_backward(s->q_raw, w[qs], dq, dq2, g[qs], n * c->heads, hd, c->eps, (int)c->norm_unit_offset);
                ops->rms_norm_backward(s->k_raw, w[ks], dk, dk2, g[ks], n * c->kv_heads, hd, c->eps, (int)c->norm_unit_offset);
            } else {
                ops->rms_norm_backward(s->q_raw, w[qs], dq, dq2, g[qs], n, qd, c->eps, (int)c->norm_unit_offset);
                ops->rms_norm_backward(s->k_raw, w[ks], dk, dk2, g[ks], n, kvd, c->eps, (int)c->norm_unit_offset);
            }
            dqf = dq2;
            dkf = dk2;
        }
        const int64_t kinds[3] = {ORC_Q, ORC_K, ORC_V};
        const int64_t biases[3] = {ORC_QB, ORC_KB, ORC_VB};
        const float* ds[3] = {dqf, dkf, dv_t};
        const int64_t outs[3] = {qd, kvd, kvd};
        for (int p = 0; p < 3; ++p) {
            const int64_t ws = orc_slot(c, l, kinds[p]);
            const int64_t bs = orc_slot(c, l, biases[p]);
            ops->linear_backward(s->h1, w[ws], ds[p], p == 0 ? dh1 : dh, g[ws], c->attn_bias ? g[bs] : NULL, n, H,
                                 outs[p]);
            if (p > 0) vadd(dh1, dh, dh1, n * H);
        }
        if (has_pre_norms(c)) {
            const int64_t an = orc_slot(c, l, ORC_ATTN_NORM);
            ops->rms_norm_backward(s->x_in, w[an], dh1, dtmp, g[an], n, H, c->eps, (int)c->norm_unit_offset);
            vadd(dx_mid, dtmp, dx, n * H);
        } else {
            vadd(dx_mid, dh1, dx, n * H);
        }
    }
    free(dh2); free(dtmp); free(dpost); free(dx_mid); free(dattended); free(dq_t); free(dk_t); free(dv_t); free(dq); free(dk);
    free(dq2); free(dk2); free(dh1); free(dh);

    /* embedding_backward, tied head (backprop.py:110-117), after the embedding multiplier's gradient */
    if (has_multiplier(c->embedding_multiplier)) vscale(dx, (float)c->embedding_multiplier, n * H);
    float* demb = falloc(V * H);
    ops->embedding_backward(dx, tokens, demb, n, H, V);
    if (c->tied) {
        vadd(demb, dhead, g[ORC_EMBEDDING], V * H);
    } else {
        memcpy(g[ORC_EMBEDDING], demb, (size_t)(V * H) * sizeof(float));
        memcpy(g[ORC_LM_HEAD], dhead, (size_t)(V * H) * sizeof(float));
    }
    free(demb);
    free(dhead);
    free(dx);
    free(grad_row);
    free_state(&st);
    return 0;
}

/* DecoderGradients.losses_and_gradients of one window (backprop.py:88-118): with a residual multiplier or a RoPE
 * attention factor the weights are folded first (_folded, backprop.py:529-537) and the gradients unfolded after (_unfold). */
int orc_window_gradients(const orc_ops* ops, const orc_config* c, float* const* w, const int64_t* tokens,
                         const int64_t* targets, int64_t n, double scale, double router_scale, float* const* g,
                         double* loss, double* router_loss_out) {
    float** owned;
    float** folded = fold_weights(c, w, &owned);
    const int rc = window_gradients(ops, c, folded ? folded : w, tokens, targets, n, scale, router_scale, g, loss,
                                    router_loss_out);
    int64_t* list = (int64_t*)malloc((size_t)(c->experts + 5) * sizeof(int64_t));
    for (int64_t l = 0; folded && rc == 0 && l < c->layers; ++l) {
        if (has_multiplier(c->residual_multiplier)) {
            const int k = residual_scaled_slots(c, l, list);
            for (int i = 0; i < k; ++i)
                vscale(g[list[i]], (float)c->residual_multiplier, orc_tensor_numel(c, list[i]));
        }
        if (has_multiplier(c->rope_attention_factor)) {
            const int k = rope_scaled_slots(c, l, list);
            for (int i = 0; i < k; ++i)
                scale_rotary_rows(c, list[i], g[list[i]], g[list[i]], (float)c->rope_attention_factor);
        }
    }
    free(list);
    free_folded(c, folded, owned);
    return rc;
}

/* _power (optimizer.py:59-63): base^exponent by repeated multiplication. */
static double power_repeated(double base, int64_t exponent) {
    double result = 1.0;
    for (int64_t i = 0; i < exponent; ++i) result *= base;
    return result;
}

int orc_train_step(const orc_ops* ops, const orc_config* c, float* const* params, float* const* m, float* const* v,
                   float* const* grads, const int64_t* order, int64_t order_len, const int64_t* tokens,
                   const int64_t* offsets, const int64_t* lengths, int64_t count, const orc_adamw* opt,
                   double* loss_out, double* norm_out) {
    const int64_t slots = orc_slot_count(c);
    float** wg = (float**)calloc((size_t)slots, sizeof(float*));
    for (int64_t s = 0; s < slots; ++s)
        if (params[s]) wg[s] = falloc(orc_tensor_numel(c, s));
    int64_t targets_total = 0;
    for (int64_t b = 0; b < count; ++b) targets_total += lengths[b] - 1;
    const double scale = 1.0 / (double)targets_total;
    double loss_total = 0.0, router_total = 0.0;
    int rc = 0;
    for (int64_t b = 0; b < count && rc == 0; ++b) {
        const int64_t* window = tokens + offsets[b];
        double loss = 0.0, rl = 0.0;
        rc = orc_window_gradients(ops, c, params, window, window + 1, lengths[b] - 1, scale,
                                  opt->router_aux_loss / (double)count, wg, &loss, &rl);
        loss_total += loss;
        router_total += rl;
        for (int64_t s = 0; s < slots; ++s) {
            if (!params[s]) continue;
            const int64_t n = orc_tensor_numel(c, s);
            if (b == 0)
                memcpy(grads[s], wg[s], (size_t)n * sizeof(float));
            else
                vadd(grads[s], wg[s], grads[s], n);
        }
    }
    for (int64_t s = 0; s < slots; ++s) free(wg[s]);
    free(wg);
    if (rc != 0) return rc;
    double total = 0.0;
    for (int64_t i = 0; i < order_len; ++i)
        total += ops->sum_squares(grads[order[i]], (size_t)orc_tensor_numel(c, order[i]));
    const double norm = sqrt(total);
    double clip = 1.0;
    if (opt->max_grad_norm > 0 && norm > opt->max_grad_norm) clip = opt->max_grad_norm / (norm + 1e-6);
    const double bc1 = 1.0 - power_repeated(opt->beta1, opt->step);
    const double bc2 = 1.0 - power_repeated(opt->beta2, opt->step);
    for (int64_t i = 0; i < order_len; ++i) {
        const int64_t s = order[i];
        const double decay = orc_tensor_ndim(c, s) >= 2 ? opt->weight_decay : 0.0;
        ops->adamw_step(params[s], grads[s], m[s], v[s], (size_t)orc_tensor_numel(c, s), opt->lr, opt->beta1,
                        opt->beta2, opt->eps, decay, bc1, bc2, clip);
    }
    double loss = loss_total / (double)targets_total;
    if (opt->router_aux_loss != 0.0) loss += opt->router_aux_loss * router_total / (double)count;
    if (loss_out) *loss_out = loss;
    if (norm_out) *norm_out = norm;
    return 0;
}
