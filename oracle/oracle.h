/*
 * CPU oracle for the fine-tuning hot path: a plain-C restatement of the reference's backward kernels, the forward
 * kernels a training step runs, its portable math, its random generator and the step orchestration.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (etalii_dllm_amd/, include/) includes, links or calls this code.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as the checker or as the CPU
 * baseline, never as the thing measured on the GPU.
 *
 * Every function cites the reference source it restates (paths relative to the reference checkout). Each output
 * element has one accumulation in double over its reduced index in ascending order, rounded to float once; products
 * of two floats are exact in double. The build uses -ffp-contract=off -fno-fast-math so every + - * / rounds once.
 */
#ifndef DLLM_ORACLE_H
#define DLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- portable math: cpp/include/dllm/math.hpp ---- */
double orc_exp(double x);     /* math.hpp:64-109 */
double orc_log(double x);     /* math.hpp:113-162 */
double orc_sin(double x);     /* math.hpp:220-232 */
double orc_cos(double x);     /* math.hpp:234-246 */
double orc_tanh(double x);    /* math.hpp:296-319 */
double orc_sigmoid(double x); /* math.hpp:322-328 */
float orc_dot(const float* a, const float* b, size_t n);                 /* math.hpp:31-37 */
size_t orc_argmax(const float* v, size_t n);                             /* math.hpp:40-53 */
void orc_softmax(const float* logits, float* out, size_t n);             /* math.hpp:387-398 */

/* ---- random: cpp/include/dllm/random.hpp ---- */
typedef struct { uint64_t s[4]; } orc_random;
void orc_random_init(orc_random* r, uint64_t seed);                      /* random.hpp:12-18 */
uint64_t orc_random_next(orc_random* r);                                 /* random.hpp:20-30 */
double orc_random_double(orc_random* r);                                 /* random.hpp:33 */
float orc_random_gaussian(orc_random* r);                                /* random.hpp:36-42 */
void orc_fill_gaussian(uint64_t seed, float* out, size_t n);             /* kernels.cpp:207-218 */

/* ---- forward kernels: cpp/include/dllm/nn.hpp ---- */
void orc_linear(const float* x, const float* w, const float* bias, float* out, size_t rows, size_t in,
                size_t out_features);                                    /* nn.hpp:28-50 */
void orc_rms_norm(const float* x, const float* w, float* out, size_t rows, size_t dim, double eps,
                  int unit_offset);                                      /* nn.hpp:391-408 */
float orc_silu(float x);                                                 /* nn.hpp:467-470 */
void orc_swiglu(const float* gate, const float* up, float* out, size_t n); /* nn.hpp:489-492 */
void orc_rope(const float* x, const int64_t* positions, const double* inv_freq, float* out, size_t tokens,
              size_t heads, size_t head_dim, size_t rotary_dim, int interleaved, int inverse); /* nn.hpp:501-530 */
void orc_attention(const float* q, const float* k, const float* v, float* out, size_t q_len, size_t kv_len,
                   size_t q_heads, size_t kv_heads, size_t head_dim, size_t value_dim, double scale, int causal,
                   size_t q_offset, size_t window, double softcap);       /* nn.hpp:535-615,729-748,870-884 */
void orc_moe_route(const float* logits, int64_t* indices, float* weights, size_t rows, size_t experts, size_t k,
                   int normalize);                                       /* nn.hpp:864-896 */

/* ---- backward kernels: cpp/include/dllm/grad.hpp ---- */
void orc_linear_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                         size_t rows, size_t in, size_t out_features);   /* grad.hpp:26-72 */
void orc_rms_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, size_t rows,
                           size_t dim, double eps, int unit_offset);     /* grad.hpp:79-111 */
float orc_silu_backward(float x, float dy);                              /* grad.hpp:177-181 */
float orc_gelu_tanh(float x);                                            /* nn.hpp:481-485 */
float orc_gelu_tanh_backward(float x, float dy);                         /* grad.hpp:183-191 */
float orc_softcap_backward(float x, float dy, double cap);               /* grad.hpp:193-197 */
void orc_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                            float* dv, size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                            size_t head_dim, size_t value_dim, double scale, int causal, size_t q_offset,
                            size_t window, double softcap);              /* grad.hpp:206-301 */
double orc_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, size_t rows, size_t vocab,
                         double scale);                                  /* grad.hpp:395-426 */
int orc_embedding_backward(const float* dy, const int64_t* tokens, float* out, size_t rows, size_t dim,
                           size_t vocab);                                /* grad.hpp:431-464 */
double orc_sum_squares(const float* v, size_t n);                        /* grad.hpp:467-473 */
void orc_adamw_step(float* param, const float* grad, float* m, float* v, size_t n, double lr, double beta1,
                    double beta2, double eps, double weight_decay, double bc1, double bc2,
                    double grad_scale);                                  /* grad.hpp:481-495 */
void orc_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights,
                            const float* dprobabilities, float* dlogits, size_t rows, size_t experts, size_t k,
                            int normalize);                              /* grad.hpp:507-541 */
void orc_column_mean(const float* x, float* out, size_t rows, size_t cols); /* interp.hpp:146-155 */
void orc_quantize_q8_0(const float* x, int8_t* q, float* scales, size_t n); /* quant.hpp:27-60 */
void orc_linear_q8(const float* x, const int8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out);                                            /* quant.hpp:143-169,355-383 */
double orc_erf(double x);                                                               /* math.hpp:345-370 */
double orc_erfc(double x);                                                              /* math.hpp:373-384 */
float orc_gelu(float x);                                                                /* nn.hpp:474-478 */
float orc_gelu_backward(float x, float dy);                                             /* grad.hpp:165-172 */
void orc_layer_norm(const float* x, const float* w, const float* b, float* out, size_t rows, size_t dim,
                    double eps);                                                        /* nn.hpp:412-432 */
void orc_layer_norm_backward(const float* x, const float* w, const float* dy, float* dx, float* dw, float* db,
                             size_t rows, size_t dim, double eps);                      /* grad.hpp:112-163 */
void orc_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out,
                          size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                          double scale);                                                /* nn.hpp:827-856 */
void orc_biased_attention_weights(const float* q, const float* k, const float* bias, float* out, size_t q_len,
                                  size_t kv_len, size_t heads, size_t head_dim, double scale);
void orc_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                   const float* dout, float* dq, float* dk, float* dv, float* dbias, size_t q_len,
                                   size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                                   double scale);                                       /* grad.hpp:300-389 */
void orc_quantize_q4_0(const float* x, uint8_t* packed, float* scales, size_t n);       /* quant.hpp:67-94 */
void orc_unpack_q4_0(const uint8_t* packed, int8_t* values, size_t n);                  /* quant.hpp:97-108 */
void orc_linear_q4(const float* x, const uint8_t* wq, const float* ws, const float* bias, float* out, size_t rows,
                   size_t in, size_t n_out);                                            /* quant.hpp:385-403 */

/* ---- rotary frequencies: src/etalii_dllm/numerics.py:267-297 (default scaling) ---- */
void orc_rope_inv_freq(size_t rotary_dim, double theta, double* out);
/* rope_inv_freq with a Hugging Face rope_scaling (numerics.py:267-349): kind 0 default, 1 linear (factor), 2 llama3
 * (factor, low_freq_factor, high_freq_factor, original_max_position_embeddings), 3 longrope (factors[i], the chosen
 * short or long set), 4 yarn (factor, original, beta_fast, beta_slow, truncate). Returns 0, or 1 for an unknown kind. */
typedef struct {
    int64_t kind;
    double factor, low_freq_factor, high_freq_factor, original, beta_fast, beta_slow;
    int64_t truncate;
    const double* factors;
} orc_rope_scaling;
int orc_rope_inv_freq_scaled(size_t rotary_dim, double theta, const orc_rope_scaling* scaling, double* out);

/* ---- the kernel table a step driver calls (the oracle's own, or the reference's through oracle/_ref) ---- */
typedef struct {
    void (*linear)(const float*, const float*, const float*, float*, size_t, size_t, size_t);
    void (*linear_backward)(const float*, const float*, const float*, float*, float*, float*, size_t, size_t, size_t);
    void (*rms_norm)(const float*, const float*, float*, size_t, size_t, double, int);
    void (*rms_norm_backward)(const float*, const float*, const float*, float*, float*, size_t, size_t, double, int);
    void (*rope)(const float*, const int64_t*, const double*, float*, size_t, size_t, size_t, size_t, int, int);
    void (*attention)(const float*, const float*, const float*, float*, size_t, size_t, size_t, size_t, size_t,
                      size_t, double, int, size_t, size_t, double);
    void (*attention_backward)(const float*, const float*, const float*, const float*, float*, float*, float*,
                               size_t, size_t, size_t, size_t, size_t, size_t, double, int, size_t, size_t, double);
    void (*silu)(const float*, float*, size_t);
    void (*swiglu)(const float*, const float*, float*, size_t);
    void (*silu_backward)(const float*, const float*, float*, size_t);
    double (*cross_entropy)(const float*, const int64_t*, float*, size_t, size_t, double);
    int (*embedding_backward)(const float*, const int64_t*, float*, size_t, size_t, size_t);
    double (*sum_squares)(const float*, size_t);
    void (*adamw_step)(float*, const float*, float*, float*, size_t, double, double, double, double, double, double,
                       double, double);
    void (*softmax)(const float*, float*, size_t);
    void (*moe_route)(const float*, int64_t*, float*, size_t, size_t, size_t, int);
    void (*moe_route_backward)(const float*, const int64_t*, const float*, const float*, float*, size_t, size_t,
                               size_t, int);
    void (*column_mean)(const float*, float*, size_t, size_t);
    float (*dot)(const float*, const float*, size_t);
    void (*gelu_tanh)(const float*, float*, size_t);
    void (*gelu_tanh_backward)(const float*, const float*, float*, size_t);
    void (*softcap)(const float*, float*, size_t, double);
    void (*softcap_backward)(const float*, const float*, float*, size_t, double);
} orc_ops;

const orc_ops* orc_default_ops(void);

/* ---- decoder configuration: src/etalii_dllm/architecture.py (the fields a decoder step reads) ---- */
typedef struct {
    int64_t vocab, hidden, inter, layers, heads, kv_heads, head_dim;
    int64_t attn_bias;   /* q/k/v biases (Qwen2) */
    int64_t qk_norm;     /* 0 none, 1 per head (Qwen3), 2 over the whole projection (OLMo 2, OLMoE) */
    int64_t window;      /* sliding window, 0 = full causal attention */
    int64_t tied;        /* lm head = token embedding */
    int64_t experts, topk, normalize, expert_inter; /* mixture of experts; experts == 0 for dense */
    int64_t rotary_dim;
    double eps, rope_theta, attention_scale;
    const double* inv_freq;        /* rotary_dim / 2 scaled inverse frequencies, or NULL for theta's defaults */
    double rope_attention_factor;  /* LongRoPE / YaRN attention factor folded into the q/k rows (1 or 0: none) */
    /* Granite's multipliers (architecture.py; 1 or 0: none): the embedding rows times embedding_multiplier, the
     * attention and MLP output projections times residual_multiplier (folded), the logits divided by logits_scaling */
    double embedding_multiplier, residual_multiplier, logits_scaling;
    /* dense_layers (architecture.py:128, 344-346): bit l set = layer l keeps a dense MLP in a model with experts
     * (Qwen3-MoE's mlp_only_layers); layers from 64 on are sparse */
    int64_t dense_layers;
    /* norm_placement (architecture.py:315-320): 0 pre (norms on each block's input), 1 post (on each block's output,
     * OLMo 2), 2 sandwich (both) */
    int64_t norm_placement;
    /* Gemma 2 and 3 (architecture.py): RMSNorm weights used as 1 + w (norm_unit_offset); activation 0 SiLU, 1 GELU with
     * the tanh approximation; full_attention_layers: bit l set = layer l ignores the sliding window (the layers not in
     * sliding_window_layers, architecture.py:353-359); local_rope_theta (0: none) rotates the windowed layers with that
     * base and no scaling (architecture.py:322-324, backprop.py:63-67); attention_softcap and logits_softcap (0: none)
     * map scores and logits s to cap tanh(s / cap) */
    int64_t norm_unit_offset, activation, full_attention_layers;
    double local_rope_theta, attention_softcap, logits_softcap;
    /* shared_expert_intermediate_size (0: none) and shared_expert_gate (architecture.py; backprop.py:308-357,
     * 501-527): a SwiGLU expert every row of a sparse layer goes through, its output times the sigmoid of a [1, hidden]
     * gate's score when gated (Qwen2-MoE), added after the routed experts */
    int64_t shared_inter, shared_gate;
    /* per-layer choices for any depth (NULL: the masks above): `layers` bytes, nonzero = dense MLP / full attention */
    const uint8_t* dense_layer_flags;
    const uint8_t* full_attention_layer_flags;
} orc_config;

/* Whether layer l's MLP is a mixture of experts (TransformerConfig.is_sparse, architecture.py:344-346). */
int orc_is_sparse(const orc_config* c, int64_t layer);

/*
 * Tensor slots. Every tensor of the decoder has a fixed slot: the globals, then per layer a block of
 * ORC_LAYER_FIXED slots followed by 3 slots per expert. Absent tensors (no bias, no QK-norm, dense vs sparse) have
 * a NULL pointer in their slot.
 */
enum {
    ORC_EMBEDDING = 0, ORC_FINAL_NORM = 1, ORC_LM_HEAD = 2, ORC_GLOBALS = 3,
    ORC_ATTN_NORM = 0, ORC_Q = 1, ORC_K = 2, ORC_V = 3, ORC_QB = 4, ORC_KB = 5, ORC_VB = 6, ORC_QNORM = 7,
    ORC_KNORM = 8, ORC_O = 9, ORC_MLP_NORM = 10, ORC_GATE = 11, ORC_UP = 12, ORC_DOWN = 13, ORC_ROUTER = 14,
    ORC_ATTN_POST_NORM = 15, ORC_MLP_POST_NORM = 16, ORC_SHARED_GATE = 17, ORC_SHARED_UP = 18, ORC_SHARED_DOWN = 19,
    ORC_SHARED_GATE_W = 20, ORC_LAYER_FIXED = 21
};
int64_t orc_layer_slots(const orc_config* c);
int64_t orc_slot_count(const orc_config* c);
int64_t orc_slot(const orc_config* c, int64_t layer, int64_t kind);            /* layer tensor */
int64_t orc_expert_slot(const orc_config* c, int64_t layer, int64_t expert, int64_t which); /* 0 gate 1 up 2 down */

/*
 * One window: loss and the gradient of every tensor (src/etalii_dllm/training/backprop.py:88-118). grads[slot] must
 * be allocated (zeroing is not required) for every present slot. Returns 0 on success. *loss gets the summed
 * cross-entropy, *router_loss the load-balancing loss (0 for dense models).
 */
int orc_window_gradients(const orc_ops* ops, const orc_config* c, float* const* w, const int64_t* tokens,
                         const int64_t* targets, int64_t n, double scale, double router_scale, float* const* grads,
                         double* loss, double* router_loss);

/* Logits [n, vocab] of the forward pass (backprop.py:69-73). */
int orc_logits(const orc_ops* ops, const orc_config* c, float* const* w, const int64_t* tokens, int64_t n,
               float* logits);

/*
 * One full fine-tuning step (training/trainer.py:290-335, training/optimizer.py:82-109): per-window gradients summed
 * in batch order, the global norm over tensors in `order` (natural name order), clipping, bias corrections by repeated
 * multiplication and AdamW per tensor (decay only for matrices). windows: `count` windows, window i has
 * lengths[i] tokens at tokens + offsets[i]. params/m/v are updated in place; grads receives the summed gradients.
 */
typedef struct {
    double lr, beta1, beta2, eps, weight_decay, max_grad_norm, router_aux_loss;
    int64_t step; /* 1-based number of this update */
} orc_adamw;

int orc_train_step(const orc_ops* ops, const orc_config* c, float* const* params, float* const* m, float* const* v,
                   float* const* grads, const int64_t* order, int64_t order_len, const int64_t* tokens,
                   const int64_t* offsets, const int64_t* lengths, int64_t count, const orc_adamw* opt,
                   double* loss_out, double* norm_out);

int64_t orc_tensor_numel(const orc_config* c, int64_t slot); /* 0 for absent slots */
int orc_tensor_ndim(const orc_config* c, int64_t slot);

#ifdef __cplusplus
}
#endif
#endif
