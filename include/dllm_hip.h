/*
 * dllm_hip: MI355X (gfx950) backend for EtAlii.Dllm's fine-tuning hot path (the backward pass and the AdamW step
 * behind `dllm finetune`), as a C ABI over hand-written HIP kernels.
 *
 * Every result is bit-identical to the reference CPU kernels (cpp/include/dllm/{nn,grad,math}.hpp of EtAlii.Dllm)
 * on the same inputs, for any batch size, row count or CU count: each output keeps the reference's one double
 * accumulation in its fixed order.
 *
 * Conventions
 *  - Array arguments are DEVICE pointers (hipMalloc'd or equivalent), C-contiguous, float32 unless stated; sizes are
 *    element counts. `stream` is a hipStream_t passed as void* (NULL = the default stream). Calls are asynchronous
 *    unless documented to return a host value.
 *  - Return value: 0 on success; 1 invalid argument (where the reference binding raises ValueError); 2 HIP error;
 *    3 out of device memory. dllm_hip_last_error() gives the calling thread's last message.
 *  - Entry points that need scratch memory take (workspace, workspace_bytes); the matching *_workspace() query gives
 *    the bytes needed. The kernel entry points never allocate; the trainer allocates once, at creation.
 *
 * Each kernel entry point names the reference interface it replaces: the Python binding in cpp/kernels.cpp and the
 * C++ kernel it wraps.
 */
#ifndef DLLM_HIP_H
#define DLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status, device plumbing (for hosts without their own GPU allocator) ---- */
const char* dllm_hip_last_error(void);
const char* dllm_hip_version(void);
int dllm_hip_device_count(int* count);
int dllm_hip_alloc(void** device_ptr, size_t bytes);
int dllm_hip_release(void* device_ptr);
int dllm_hip_upload(void* device_dst, const void* host_src, size_t bytes);
int dllm_hip_download(void* host_dst, const void* device_src, size_t bytes);
int dllm_hip_memset(void* device_ptr, int value, size_t bytes);
int dllm_hip_synchronize(void);
/* Device-to-device copy on `stream` (asynchronous): the library's own streaming kernel. */
int dllm_hip_copy(void* device_dst, const void* device_src, size_t bytes, void* stream);

/* ---- forward kernels ---- */

/* linear: out[rows, out_f] = x[rows, in_f] @ weight[out_f, in_f]^T (+ bias); k ascending in double, bias added before
 * the one rounding. Replaces kernels.cpp:220-238 `linear` (nn.hpp:28-50, 348-359). */
size_t dllm_hip_linear_workspace(size_t rows, size_t in_features, size_t out_features);
int dllm_hip_linear(const float* x, const float* weight, const float* bias, float* out, size_t rows,
                    size_t in_features, size_t out_features, void* workspace, size_t workspace_bytes, void* stream);

/* rms_norm over the last dimension (weight may be NULL). Replaces kernels.cpp:598-611 `rms_norm` (nn.hpp:391-408). */
int dllm_hip_rms_norm(const float* x, const float* weight, float* out, size_t rows, size_t dim, double eps,
                      int add_unit_offset, void* stream);

/* rope of x[tokens, heads, head_dim] at positions (int64) with inv_freq (double, rotary_dim / 2 entries).
 * Replaces kernels.cpp:662-679 `rope` (nn.hpp:501-530); inverse = 1 is the RoPE backward. */
size_t dllm_hip_rope_workspace(size_t tokens, size_t rotary_dim);
int dllm_hip_rope(const float* x, const int64_t* positions, const double* inv_freq, float* out, size_t tokens,
                  size_t heads, size_t head_dim, size_t rotary_dim, int interleaved, int inverse, void* workspace,
                  size_t workspace_bytes, void* stream);

/* rope_inv_freq (numerics.py:267-349, a host function): rotary_dim / 2 inverse frequencies theta^(-2i / rotary_dim)
 * from the portable exp and log (rotary_dim 0: head_dim), with a Hugging Face rope_scaling: kind 0 default, 1 linear
 * (factor), 2 llama3 (factor, low/high_freq_factor, original_max_position_embeddings), 3 longrope (factors: the
 * chosen short or long set, one per pair), 4 yarn (factor, original_max_position_embeddings, beta_fast, beta_slow,
 * truncate). Same bits as the reference's Python double arithmetic. */
typedef struct {
    int64_t kind;
    double factor, low_freq_factor, high_freq_factor, original_max_position_embeddings, beta_fast, beta_slow;
    int64_t truncate;
    const double* factors;
} dllm_hip_rope_scaling;
int dllm_hip_rope_inv_freq(size_t head_dim, double theta, size_t rotary_dim, const dllm_hip_rope_scaling* scaling,
                           double* out);

/* Causal / windowed grouped-query attention, q[q_len, q_heads, head_dim], k[kv_len, kv_heads, head_dim],
 * v[kv_len, kv_heads, value_dim] -> out[q_len, q_heads, value_dim]; q_offset < 0 means kv_len - q_len.
 * Replaces kernels.cpp:680-705 `attention` (nn.hpp:761-796). Any key length. Self-attention shapes (q_len == kv_len,
 * no cached prefix, no soft-cap, head_dim == value_dim a multiple of 4; causal, or non-causal without a window) run on
 * the training step's matrix-core tiles, with a workspace of about q_heads * q_len^2 doubles (four times that for the
 * backward); other shapes run one wave per (query, head). Both give the reference's bits. The workspace functions
 * take the call's shape arguments. */
size_t dllm_hip_attention_workspace(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads, size_t head_dim,
                                    size_t value_dim, int causal, int64_t q_offset, size_t window, double softcap);
int dllm_hip_attention(const float* q, const float* k, const float* v, float* out, size_t q_len, size_t kv_len,
                       size_t q_heads, size_t kv_heads, size_t head_dim, size_t value_dim, double scale, int causal,
                       int64_t q_offset, size_t window, double softcap, void* workspace, size_t workspace_bytes,
                       void* stream);

/* silu elementwise (kernels.cpp:628, nn.hpp:467-470), gelu_tanh elementwise (kernels.cpp:632, nn.hpp:481-485) and
 * swiglu = f32(act(gate)) * up with act silu (kind 0) or gelu_tanh (kind 2); another kind is an invalid argument
 * (kernels.cpp:633-649, nn.hpp:488-492). */
int dllm_hip_silu(const float* x, float* out, size_t n, void* stream);
int dllm_hip_gelu_tanh(const float* x, float* out, size_t n, void* stream);
int dllm_hip_swiglu(const float* gate, const float* up, float* out, size_t n, int kind, void* stream);
/* f32(cap tanh(x / cap)) elementwise in double; cap > 0. Replaces kernels.cpp:650-660 `softcap` (nn.hpp:457-461). */
int dllm_hip_softcap(const float* x, float* out, size_t n, double cap, void* stream);
/* f32(sigmoid(x)) elementwise with the portable sigmoid. Replaces kernels.cpp:629-630 `sigmoid_elementwise`
 * (nn.hpp:464, math.hpp:322-328). */
int dllm_hip_sigmoid_elementwise(const float* x, float* out, size_t n, void* stream);

/* ---- backward kernels ---- */

/* (dx, dweight, dbias) of linear; dx, dweight, dbias may each be NULL. Replaces kernels.cpp:811-837
 * `linear_backward` (grad.hpp:26-72). */
size_t dllm_hip_linear_backward_workspace(size_t rows, size_t in_features, size_t out_features);
int dllm_hip_linear_backward(const float* x, const float* weight, const float* dy, float* dx, float* dweight,
                             float* dbias, size_t rows, size_t in_features, size_t out_features, void* workspace,
                             size_t workspace_bytes, void* stream);

/* (dx, dweight) of rms_norm; dweight may be NULL. Replaces kernels.cpp:839-856 `rms_norm_backward`
 * (grad.hpp:79-111). */
size_t dllm_hip_rms_norm_backward_workspace(size_t rows);
int dllm_hip_rms_norm_backward(const float* x, const float* weight, const float* dy, float* dx, float* dweight,
                               size_t rows, size_t dim, double eps, int add_unit_offset, void* workspace,
                               size_t workspace_bytes, void* stream);

/* dy * silu'(x) elementwise. Replaces kernels.cpp:890-901 `silu_backward` (grad.hpp:177-181). */
int dllm_hip_silu_backward(const float* x, const float* dy, float* out, size_t n, void* stream);
/* dy * gelu_tanh'(x) elementwise. Replaces kernels.cpp:903-914 `gelu_tanh_backward` (grad.hpp:183-191). */
int dllm_hip_gelu_tanh_backward(const float* x, const float* dy, float* out, size_t n, void* stream);
/* dy * softcap'(x) = dy (1 - tanh(x / cap)^2) elementwise; cap > 0. Replaces kernels.cpp:916-928
 * `softcap_backward` (grad.hpp:193-197). */
int dllm_hip_softcap_backward(const float* x, const float* dy, float* out, size_t n, double cap, void* stream);

/* (dq, dk, dv) of attention. Replaces kernels.cpp:930-959 `attention_backward` (grad.hpp:206-301). */
size_t dllm_hip_attention_backward_workspace(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                                             size_t head_dim, size_t value_dim, int causal, int64_t q_offset,
                                             size_t window, double softcap);
int dllm_hip_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq,
                                float* dk, float* dv, size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads,
                                size_t head_dim, size_t value_dim, double scale, int causal, int64_t q_offset,
                                size_t window, double softcap, void* workspace, size_t workspace_bytes, void* stream);

/* Softmax cross-entropy of logits[rows, vocab] against int64 targets (negative = ignored): dlogits * scale, and the
 * summed loss written to *loss (HOST pointer; the call waits for the stream). A target >= vocab is an invalid
 * argument, as in the reference. Replaces kernels.cpp:991-1003 `cross_entropy` (grad.hpp:395-426). */
size_t dllm_hip_cross_entropy_workspace(size_t rows);
int dllm_hip_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, size_t rows, size_t vocab,
                           double scale, double* loss, void* workspace, size_t workspace_bytes, void* stream);

/* Embedding gradient out[vocab, dim]: dy rows summed per token id in position order. Reads the token ids back to the
 * host to group them (the call waits for the stream); an id outside [0, vocab) is an invalid argument.
 * Replaces kernels.cpp:1029-1039 `embedding_backward` (grad.hpp:431-464). */
size_t dllm_hip_embedding_backward_workspace(size_t rows);
int dllm_hip_embedding_backward(const float* dy, const int64_t* tokens, float* out, size_t rows, size_t dim,
                                size_t vocab, void* workspace, size_t workspace_bytes, void* stream);

/* Sum of squares in index order with a double accumulator, written to *result (HOST pointer; waits): the bits of the
 * serial chain, computed in parallel (each add within one binade of the running sum is an integer increment plus a
 * parity-dependent rounding bit, composed as an associative scan; binade changes are replayed as real adds).
 * Replaces kernels.cpp:1041-1043 `sum_squares` (grad.hpp:467-473). */
size_t dllm_hip_sum_squares_workspace(size_t n);
int dllm_hip_sum_squares(const float* values, size_t n, double* result, void* workspace, size_t workspace_bytes,
                         void* stream);

/* sum_squares without a workspace and without any allocation: the same bits as dllm_hip_sum_squares, its scratch
 * (plan, block sums, block functions, result) in a fixed 4 MiB device array that each GPU holds until the process
 * ends. n is at most 2^29 (larger is an invalid argument, refused before any launch). Calls on one GPU are
 * serialised on that array (a per-GPU lock held until the call's stream has finished). No counterpart in the reference: it is for callers that cannot allocate device memory (code
 * under graph capture, tight serving loops, harnesses that forbid hipMalloc). Waits for the stream. */
int dllm_hip_sum_squares_noalloc(const float* values, size_t n, double* result, void* stream);

/* One in-place AdamW step. Replaces kernels.cpp:1045-1057 `adamw_step` (grad.hpp:481-495). */
int dllm_hip_adamw_step(float* param, const float* grad, float* m, float* v, size_t n, double lr, double beta1,
                        double beta2, double eps, double weight_decay, double bias_correction1,
                        double bias_correction2, double grad_scale, void* stream);

/* ---- mixture-of-experts routing ---- */

/* indices [rows, k] (int64) and weights [rows, k] of MoE routing: each row's softmax, the k largest probabilities in
 * a total order (ties to the lower expert), divided by their total with normalize; rank order. Replaces
 * kernels.cpp:190-204 `moe_route` (nn.hpp:864-896). k outside [1, experts] is an invalid argument. */
int dllm_hip_moe_route(const float* logits, int64_t* indices, float* weights, size_t rows, size_t experts, size_t k,
                       int normalize, void* stream);
/* dlogits [rows, experts] from the gradients of the routing weights dweights [rows, k] and (optional, may be NULL)
 * of the softmax probabilities dprobabilities [rows, experts]. Replaces kernels.cpp:1005-1027
 * `moe_route_backward` (grad.hpp:507-541). */
int dllm_hip_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights,
                                const float* dprobabilities, float* dlogits, size_t rows, size_t experts, size_t k,
                                int normalize, void* stream);

/* softmax of each of rows vectors of n logits (rows = 1 is the binding). Replaces kernels.cpp:166-176 `softmax`
 * (math.hpp:387-398). */
int dllm_hip_softmax(const float* logits, float* out, size_t rows, size_t n, void* stream);
/* out[c] = f32(sum over rows ascending of x[r][c] in double / rows). Replaces kernels.cpp:787-796 `column_mean`
 * (interp.hpp:146-155). */
int dllm_hip_column_mean(const float* x, float* out, size_t rows, size_t cols, void* stream);
/* *result (HOST) = f32(sum over i ascending of a[i] b[i] in double); waits. The workspace holds one float
 * (dllm_hip_dot_workspace). Replaces kernels.cpp:153-161 `dot` (math.hpp:31-37). */
size_t dllm_hip_dot_workspace(void);
int dllm_hip_dot(const float* a, const float* b, size_t n, float* result, void* workspace, size_t workspace_bytes,
                 void* stream);

/* ---- LoRA on a frozen (optionally Q8_0) base ---- */

/* quantize_q8_0 of n values (a multiple of 32): int8 values and one float scale per 32-value block. Replaces
 * kernels.cpp's `quantize_q8_0` binding (quant.hpp:27-60) as QuantizedWeight uses it (numerics.py:122-124). */
int dllm_hip_quantize_q8_0(const float* x, int8_t* q, float* scales, size_t n, void* stream);
/* out = f32(q) * scale of the value's block. Replaces QuantizedWeight.dequantize (numerics.py:138-139). */
int dllm_hip_dequantize_q8_0(const int8_t* q, const float* scales, float* out, size_t n, void* stream);

/* ---- encoder and T5 training kernels (cpp/include/dllm/grad.hpp:112-174, 300-389; nn.hpp:412-432, 474-478,
 * 827-856) ----
 * gelu / gelu_backward: kernels.cpp:631, 877-889 (exact erf GELU with the portable erfc). layer_norm /
 * layer_norm_backward: kernels.cpp:612-625, 858-875 (dx, dw, db; dw and db summed over all rows in order; any of the
 * three outputs may be NULL). biased_attention / biased_attention_backward: kernels.cpp:707-727, 961-990 (T5's
 * attention with bias [heads, q_len, kv_len]; q [q_len, heads, head_dim], k [kv_len, heads, head_dim], v [kv_len,
 * heads, value_dim]; returns dq, dk, dv, dbias). Self-attention shapes (q_len == kv_len, head_dim and value_dim
 * multiples of 4) run on the matrix-core tiles, with a larger workspace; the results are the same bits either way. */
int dllm_hip_gelu(const float* x, float* out, size_t n, void* stream);
int dllm_hip_gelu_backward(const float* x, const float* dy, float* out, size_t n, void* stream);
int dllm_hip_layer_norm(const float* x, const float* weight, const float* bias, float* out, size_t rows, size_t dim,
                        double eps, void* stream);
size_t dllm_hip_layer_norm_backward_workspace(size_t rows);
int dllm_hip_layer_norm_backward(const float* x, const float* weight, const float* dy, float* dx, float* dw,
                                 float* db, size_t rows, size_t dim, double eps, void* workspace,
                                 size_t workspace_bytes, void* stream);
size_t dllm_hip_biased_attention_workspace(size_t q_len, size_t kv_len, size_t heads, size_t head_dim,
                                           size_t value_dim);
int dllm_hip_biased_attention(const float* q, const float* k, const float* v, const float* bias, float* out,
                              size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                              double scale, void* workspace, size_t workspace_bytes, void* stream);
/* biased_attention_weights (kernels.cpp:753-773, interp.hpp:79-121): the probabilities [q_len, heads, kv_len] of
 * biased_attention, f32(e (1 / total)); workspace: dllm_hip_biased_attention_workspace(q_len, kv_len, heads,
 * head_dim, 4). */
int dllm_hip_biased_attention_weights(const float* q, const float* k, const float* bias, float* out, size_t q_len,
                                      size_t kv_len, size_t heads, size_t head_dim, double scale, void* workspace,
                                      size_t workspace_bytes, void* stream);
size_t dllm_hip_biased_attention_backward_workspace(size_t q_len, size_t kv_len, size_t heads, size_t head_dim,
                                                    size_t value_dim);
int dllm_hip_biased_attention_backward(const float* q, const float* k, const float* v, const float* bias,
                                       const float* dout, float* dq, float* dk, float* dv, float* dbias,
                                       size_t q_len, size_t kv_len, size_t heads, size_t head_dim, size_t value_dim,
                                       double scale, void* workspace, size_t workspace_bytes, void* stream);

/* ---- quantised linear layers for inference (cpp/include/dllm/quant.hpp:143-169, 355-403; kernels.cpp:310-385) ----
 * linear_q8: x [rows, in] quantised to Q8_0 per row block of 32, q [out, in] int8 (8-byte aligned) and scales
 * [out, in / 32]; out[r][n] = f32(sum over blocks ascending of (f64(xs) f64(ws)) f64(isum) + bias[n]), isum the
 * exact int32 dot of a block (replaces kernels.cpp:310-329 `linear_q8`). in must be a multiple of 32. */
size_t dllm_hip_linear_q8_workspace(size_t rows, size_t in);
int dllm_hip_linear_q8(const float* x, const int8_t* q, const float* scales, const float* bias, float* out,
                       size_t rows, size_t in, size_t out_f, void* workspace, size_t workspace_bytes, void* stream);
/* Q4_0 (kernels.cpp:331-385): quantize_q4_0 of n floats into n / 2 packed bytes and n / 32 scales; unpack_q4_0 to
 * int8; linear_q4 = linear_q8 of the unpacked weights. */
int dllm_hip_quantize_q4_0(const float* x, uint8_t* packed, float* scales, size_t n, void* stream);
int dllm_hip_unpack_q4_0(const uint8_t* packed, int8_t* values, size_t n, void* stream);
size_t dllm_hip_linear_q4_workspace(size_t rows, size_t in, size_t out);
int dllm_hip_linear_q4(const float* x, const uint8_t* q, const float* scales, const float* bias, float* out,
                       size_t rows, size_t in, size_t out_f, void* workspace, size_t workspace_bytes, void* stream);
/* out = weight + f32(linear(b, a^T)) * f32(scale) for weight [out_f, in_f], a [rank, in_f], b [out_f, rank].
 * Replaces lora.merge (src/etalii_dllm/lora.py:271-276). */
size_t dllm_hip_lora_merge_workspace(size_t out_features, size_t in_features, size_t rank);
int dllm_hip_lora_merge(const float* weight, const float* a, const float* b, float* out, size_t out_features,
                        size_t in_features, size_t rank, double scale, void* workspace, size_t workspace_bytes,
                        void* stream);
/* da = f32(linear(b^T, grad^T)) * f32(scale), db = f32(linear(grad, a)) * f32(scale) from the merged weight's
 * gradient grad [out_f, in_f]. Replaces lora.adapter_gradients (src/etalii_dllm/lora.py:374-383). */
size_t dllm_hip_lora_adapter_gradients_workspace(size_t out_features, size_t in_features, size_t rank);
int dllm_hip_lora_adapter_gradients(const float* grad, const float* a, const float* b, float* da, float* db,
                                    size_t out_features, size_t in_features, size_t rank, double scale,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* ---- the device-resident fine-tuning step ----
 *
 * Replaces the Python step the reference runs through those kernels: FineTuner.train_step
 * (src/etalii_dllm/training/trainer.py:290-335) over DecoderGradients (training/backprop.py:88-118, 183-357, 399-527)
 * and AdamW.step (training/optimizer.py:82-109). Weights, gradients, AdamW moments and every activation stay in
 * device memory; all windows of a step run as one packed batch (row-local work is batch-invariant), and every
 * reduction over a window's rows is kept per window and summed across windows in float in window order, exactly
 * as the reference sums its per-window gradient sets.
 */
typedef struct {
    int64_t vocab, hidden, intermediate, layers, heads, kv_heads, head_dim;
    int64_t attention_bias;   /* q/k/v biases (Qwen2) */
    int64_t qk_norm;          /* 0 none, 1 per head (Qwen3), 2 whole projection (OLMo 2) */
    int64_t sliding_window;   /* 0 = full causal attention */
    int64_t tie_embeddings;
    int64_t experts, experts_per_token, normalize_expert_weights, expert_intermediate; /* 0 experts: dense */
    int64_t rotary_dim;
    double rms_norm_eps, rope_theta, attention_scale;
    /* Granite's multipliers (architecture.py TransformerConfig; 0 or 1: none): the embedding rows times
     * embedding_multiplier (backprop.py:418-419), the attention and MLP outputs times residual_multiplier (folded into
     * the output and down projections, transformer.py:231-239), the logits divided by logits_scaling
     * (backprop.py:174-181). Granite's attention_multiplier is attention_scale. */
    double embedding_multiplier, residual_multiplier, logits_scaling;
    /* dense_layers (architecture.py:128, 344-346; Qwen3-MoE's mlp_only_layers): bit l set = layer l keeps a dense
     * MLP of `intermediate` in a model with experts; layers from 64 on are routed (dense_layer_flags below reaches
     * any depth) */
    int64_t dense_layers;
    /* norm_placement (architecture.py:315-320): 0 pre (RMSNorm on each block's input), 1 post (on each block's
     * output before the residual add, OLMo 2), 2 both; with routed experts too */
    int64_t norm_placement;
    /* Gemma 2 and 3 (architecture.py, importer.py:283-345): norms with 1 + w (norm_unit_offset); the MLP's activation
     * 0 SiLU, 1 GELU-tanh; full_attention_layers: bit l set = layer l ignores sliding_window (the layers outside
     * sliding_window_layers); local_rope_theta (0: none) rotates the windowed layers with that base and no scaling;
     * attention_softcap and logits_softcap (0: none) map each scaled score and each logit x to cap tanh(x / cap). */
    int64_t norm_unit_offset, activation, full_attention_layers;
    double local_rope_theta, attention_softcap, logits_softcap;
    /* A shared expert in every routed layer (architecture.py shared_expert_intermediate_size, shared_expert_gate;
     * backprop.py:308-357, 501-527): shared_inter (0: none) is its SwiGLU size; every row goes
     * through it, and with shared_gate its output is multiplied by the sigmoid of a [1, hidden] gate's score (Qwen2-MoE);
     * its output is added after the routed experts'. */
    int64_t shared_inter, shared_gate;
    /* Per-layer choices for models of any depth (NULL: the masks above, which reach layers 0-63 only): `layers`
     * bytes each, nonzero = layer l keeps a dense MLP (dense_layers) / ignores sliding_window (full attention).
     * Read at creation only. */
    const uint8_t* dense_layer_flags;
    const uint8_t* full_attention_layer_flags;
} dllm_hip_decoder_config;

typedef struct dllm_hip_trainer dllm_hip_trainer;

/* Allocates every buffer for steps of up to max_tokens tokens (rows, summed over windows) in up to max_windows
 * windows, each at most max_window_tokens long. Weights start at zero; moments at zero. */
/* LoRA runs (src/etalii_dllm/lora.py, training/trainer.py:463-474): AdamW updates the adapters only. Targets are a
 * mask of q (1) k (2) v (4) o (8) gate (16) up (32) down (64); scale = alpha / rank (alpha / sqrt(rank) with
 * rslora). base_quantize 1 (q8_0) or 2 (q4_0) holds the quantisable matrices (lora.py:319-324) as their dequantised
 * values, applied at the step after the parameters are written (QuantizedBase: a quantised run is LoRA on the
 * dequantised base, lora.py:327-375). */
typedef struct {
    int64_t rank;
    double alpha;
    int64_t targets;
    int64_t rslora;
    int64_t base_quantize;
} dllm_hip_lora_config;

int dllm_hip_trainer_create(const dllm_hip_decoder_config* config, int64_t max_tokens, int64_t max_windows,
                            int64_t max_window_tokens, dllm_hip_trainer** trainer);
int dllm_hip_trainer_destroy(dllm_hip_trainer* trainer);
/* A LoRA trainer (lora may be NULL: as dllm_hip_trainer_create). The adapters are tensors "<weight>.lora_a"
 * ([rank, in]) and "<weight>.lora_b" ([out, rank]) beside the base tensors; set them (init_adapters) before the first
 * step. The adapted base tensors' gradients (which 1) are those of the merged weights; the other base tensors'
 * gradients reach no optimizer and are not computed (they stay zero). No counterpart in the reference's
 * kernel module: it replaces FineTuner's LoRA branch (trainer.py:247-250, 304-305). */
int dllm_hip_trainer_create_lora(const dllm_hip_decoder_config* config, const dllm_hip_lora_config* lora,
                                 int64_t max_tokens, int64_t max_windows, int64_t max_window_tokens,
                                 dllm_hip_trainer** trainer);

/* The device buffer of one tensor, by the reference's tensor name (architecture.py:418-468), e.g.
 * "layers.3.attention.q.weight": which = 0 parameter, 1 gradient (of the last step), 2 first moment, 3 second moment.
 * Parameters written through this pointer take effect at the next step. */
int dllm_hip_trainer_tensor(dllm_hip_trainer* trainer, const char* name, int which, float** device_ptr,
                            int64_t* numel);
/* The rotary inverse frequencies (rotary_dim / 2 values, host array: dllm_hip_rope_inv_freq with the model's scaling)
 * and the LongRoPE / YaRN attention factor (architecture.py:331-336; 1 for none) of the next steps. The factor is
 * folded into the rows of the q and k projections (and biases) feeding the rotated dimensions, or into the QK-norm
 * weights' rotated entries when the model has QK-norm (fold_scales, transformer.py:204-245), and each window's
 * gradients of those tensors are multiplied by it again (_unfold, backprop.py:380-394). Without this call a trainer
 * uses theta's default frequencies and no factor. No counterpart in the kernel module: DecoderGradients reads both
 * from the TransformerConfig. */
int dllm_hip_trainer_set_rope(dllm_hip_trainer* trainer, const double* inv_freq, int64_t pairs,
                              double attention_factor);
/* Tensor names in natural order (modelfile.py:40-47); index in [0, count). */
int dllm_hip_trainer_tensor_count(dllm_hip_trainer* trainer, int64_t* count);
const char* dllm_hip_trainer_tensor_name(dllm_hip_trainer* trainer, int64_t index);

/* Gradients only (DecoderGradients.losses_and_gradients summed over windows in batch order): tokens is a HOST int64
 * array; window w is tokens[offsets[w] .. offsets[w] + lengths[w]) and predicts its own next tokens (inputs are the
 * first lengths[w] - 1 tokens). scale multiplies the summed cross-entropy; *loss (host) receives the summed loss.
 * router_scale multiplies each window's router load-balancing loss in the gradients (routed experts; backprop.py
 * 359-377); the summed router loss of the call is read with dllm_hip_trainer_router_loss. */
int dllm_hip_trainer_gradients(dllm_hip_trainer* trainer, const int64_t* tokens, const int64_t* offsets,
                               const int64_t* lengths, int64_t windows, double scale, double router_scale,
                               double* loss, void* stream);
/* The router loss summed over the windows of the last gradients or step call (0 for dense models). No counterpart in
 * the kernel module: it is the second value of losses_and_gradients (backprop.py:88-118) summed as trainer.py:327. */
int dllm_hip_trainer_router_loss(dllm_hip_trainer* trainer, double* router_loss);

typedef struct {
    double learning_rate, beta1, beta2, eps, weight_decay, max_grad_norm, router_aux_loss;
    int64_t step; /* 1-based number of this update */
} dllm_hip_adamw;

/* One full step: gradients with scale 1 / (sum of lengths - windows) and router_scale router_aux_loss / windows, the
 * global norm, clipping and AdamW in natural tensor order. *loss gets the mean loss plus router_aux_loss times the mean
 * router loss (trainer.py:312-335), *grad_norm the norm before clipping (host pointers; waits). */
int dllm_hip_trainer_step(dllm_hip_trainer* trainer, const int64_t* tokens, const int64_t* offsets,
                          const int64_t* lengths, int64_t windows, const dllm_hip_adamw* adamw, double* loss,
                          double* grad_norm, void* stream);

/* One direct-preference-optimization step (FineTuner._preference_gradients, trainer.py:364-384, then the update of
 * trainer.py:303-306). Windows 2p and 2p + 1 are pair p's tokens prompt + chosen answer and prompt + rejected answer
 * (PreferencePair.sequence, preference.py:97-102); their first prompt_lengths[p] - 1 targets are not scored.
 * reference holds the reference model's log-probabilities, [pairs][chosen, rejected]. With z = beta ((-l_c - r_c) -
 * (-l_r - r_r)) from the windows' summed cross-entropies l, the gradient is the window-ordered float sum of each
 * window's gradient times f32(beta (1 - sigmoid(z)) / pairs) (minus that for the rejected answer); *loss is the mean
 * of -log_sigmoid(z) over the pairs, *grad_norm the norm before clipping (host pointers; waits). */
int dllm_hip_trainer_dpo_step(dllm_hip_trainer* trainer, const int64_t* tokens, const int64_t* offsets,
                              const int64_t* lengths, const int64_t* prompt_lengths, int64_t pairs,
                              const double* reference, double beta, const dllm_hip_adamw* adamw, double* loss,
                              double* grad_norm, void* stream);
/* Minus each window's summed cross-entropy with its first prompt_lengths[w] - 1 targets not scored: an answer's
 * log-probability after its prompt (FineTuner.log_probability, trainer.py:443-453); out is a host array. */
int dllm_hip_trainer_log_probabilities(dllm_hip_trainer* trainer, const int64_t* tokens, const int64_t* offsets,
                                       const int64_t* lengths, const int64_t* prompt_lengths, int64_t windows,
                                       double* out, void* stream);

/* Matmul timing inside steps: with profiling on, every matmul launch of the trainer is bracketed by HIP events on its
 * stream; _read sums them (waiting for the events) into the number of launches, their total milliseconds and their
 * algorithmic flops (2 * rows * columns * reduction length each). Enabling resets the totals. */
int dllm_hip_trainer_profile(dllm_hip_trainer* trainer, int enable);
int dllm_hip_trainer_profile_read(dllm_hip_trainer* trainer, int64_t* launches, double* milliseconds, double* flops);

/* ---- model and checkpoint files (src/etalii_dllm/modelfile.py, training/trainer.py:477-630) ----
 * kind 0: model.dllm (write_model_file, modelfile.py:68-136): prefix "DLLM", u32 1, u64 header length; the data
 *   section is weights() (trainer.py:460-468; LoRA targets merged) in natural order.
 * kind 1: .dllmckpt (FineTuner.save_checkpoint, trainer.py:524-568): prefix "DLLMCKPT", u32 1, u64 header length;
 *   the data section is param/<name> for the trained tensors, then adam_m/<name>, adam_v/<name> per tensor.
 * Every tensor is float32, padded with zeros to 64 bytes; the fingerprint is the SHA-256 of the data section
 * (modelfile.data_fingerprint, modelfile.py:228-235, for kind 0). hex_out receives 64 hex digits and a NUL. */

/* The fingerprint of a trainer's current data section, streamed from device memory (waits). Replaces
 * modelfile.data_fingerprint(FineTuner.weights()) and the checkpoint's data hash without a host copy. */
int dllm_hip_trainer_fingerprint(dllm_hip_trainer* trainer, int kind, char* hex_out, void* stream);
/* Writes a file: header is the caller's canonical JSON (modelfile.canonical_json of the header dict, with
 * "fingerprint" set to 64 zeros, unpadded); the library pads it with spaces so the data starts at a multiple of 64,
 * streams the data section from device memory and patches the fingerprint into the header. Same bytes as
 * write_model_file / save_checkpoint for the same header. */
int dllm_hip_trainer_write_file(dllm_hip_trainer* trainer, int kind, const char* path, const char* header,
                                size_t header_len, char* hex_out, void* stream);
/* Restores the trained tensors and both moments from a checkpoint (FineTuner.load_checkpoint, trainer.py:570-630):
 * the data section's SHA-256 must equal `fingerprint` (the header's, 64 hex digits) or status 1 is returned and
 * nothing is loaded. The caller checks the header (data fingerprint, base model, tensor list). */
int dllm_hip_trainer_read_checkpoint(dllm_hip_trainer* trainer, const char* path, const char* fingerprint,
                                     void* stream);
/* Host-only helpers (no GPU): SHA-256 of a buffer (impl 0 fastest, 1 portable, 2 x86 SHA extensions when present);
 * a tensor file from host arrays (the layout above); the SHA-256 of a file's data section. No counterpart in the
 * kernel module: hashlib.sha256, write_model_file with host tensors, and ModelFile.verify's hash. */
int dllm_hip_sha256(const void* data, size_t n, int impl, char* hex_out);
int dllm_hip_write_tensor_file(const char* path, int kind, const char* header, size_t header_len,
                               const float* const* host_tensors, const int64_t* numels, size_t count, char* hex_out);
int dllm_hip_tensor_file_fingerprint(const char* path, int kind, char* hex_out);

/* ---- seeded synthetic inputs (kernels.cpp:130-136 `Random`, kernels.cpp:206-218 `fill_gaussian`) ----
 * Host functions: n Irwin-Hall Gaussians of Random(seed), times scale (one float multiply; 1 keeps them as is), and
 * n token ids Random(seed).next_u64() % vocab. */
int dllm_hip_fill_gaussian(uint64_t seed, float* host_out, size_t n, float scale);
int dllm_hip_random_tokens(uint64_t seed, int64_t* host_out, size_t n, int64_t vocab);

#ifdef __cplusplus
}
#endif
#endif
