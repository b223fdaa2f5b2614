// Internal launchers of the HIP kernels (device pointers, explicit sizes, one stream). The C-ABI in capi.hip and the
// device-resident trainer in trainer.hip are built on these; nothing here allocates.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dllm_hip {

// ---- matmuls (gemm.hip) ----

// Rows of the double operand are padded to whole row tiles: lda >= padded_rows(I).
int64_t padded_rows(int64_t n);

struct GemmCall {
    const double* A = nullptr;  // [L][lda] doubles, i contiguous (a_kind 0)
    int64_t lda = 0;            // row stride of A, or of Af
    const float* Af = nullptr;  // a_kind 1: Af[l][i] = A[l][i]; a_kind 2: Af[i][l] = A[l][i] (plain mode, l1 % 4 == 0)
    int a_kind = 0;
    const float* B = nullptr;  // [L][ldb] floats, j contiguous
    int64_t ldb = 0;
    float* C = nullptr;  // [I][ldc]
    int64_t ldc = 0;
    int64_t I = 0, J = 0;
    int64_t l0 = 0, l1 = 0;            // plain mode: reduce over l in [l0, l1)
    const int64_t* seg = nullptr;      // segmented mode (device): nseg + 1 offsets; C = window-ordered float sum
    int nseg = 1;
    const float* bias = nullptr;       // plain: + bias[j] in double before rounding
    const float* addsrc = nullptr;     // plain: C = addsrc[i][j] + f32(sum) (may alias C)
    int64_t ld_add = 0;
    const float* seg_addend = nullptr; // segmented: per-window addend rows
    const int* seg_addrow = nullptr;   // [nseg][I] rows into seg_addend, -1 for none
    int64_t ld_seg_add = 0;
    // segmented: optional scratch of seg_partial_cap floats; when nseg * I * J fit and the tile grid is small, the
    // windows run in parallel into it and a second pass adds them in window order
    float* seg_partial = nullptr;
    int64_t seg_partial_cap = 0;
    // segmented, float A rows: optional per-window float factors (device, nseg): window s adds f32(result * w[s])
    const float* seg_weight = nullptr;
    // segmented, float A rows: optional per-row float factors (device, I): row i of each window's result times
    // rowscale[i], before the window factor (the RoPE attention factor's unfold of a window's gradient)
    const float* seg_rowscale = nullptr;
    // float A in a shape the matrix-core kernel cannot stage: when given, A is widened into this double scratch
    // (a_scratch_cap doubles, at least l1 x padded_rows(I)) and the call runs on the VALU kernels with the same bits
    double* a_scratch = nullptr;
    int64_t a_scratch_cap = 0;
};
// Whether a float-A call runs on the matrix-core kernel (every operand row a whole number of 16-byte chunks).
bool gemm_mfma_shape(const GemmCall& g);

int launch_gemm(const GemmCall& g, hipStream_t stream);

// Several independent matmuls in one launch (the experts of a layer). All are float-A of one kind: transposed
// (plain mode) or rows (plain or windowed, no addends). gemm_group_prepare lays the parameters of n <= capacity calls
// out in host_table (gemm_group_bytes(capacity) bytes; calls with no output are dropped); the caller copies that
// table to device memory and launches it with launch_gemm_group. Each output is bit-identical to launch_gemm of its
// call.
struct GemmGroup {
    int count = 0, capacity = 0, a_kind = 0, segmented = 0;
    int tile = 4;                 // workgroup tiles of 32 tile x 32 tile outputs
    int64_t tiles = 0, grid = 0;  // grid: workgroups of the launch (8 XCD ranges of equal work, padded)
};
size_t gemm_group_bytes(int n);
int gemm_group_prepare(const GemmCall* calls, int n, int capacity, void* host_table, GemmGroup* group);
int launch_gemm_group(const GemmGroup& group, const void* device_table, hipStream_t stream);
// Row groups: matmul k of the group reads and writes rows [start[k], start[k + 1]) of shared grouped operands, the
// starts in device memory (the routed experts, grouped on the device). gemm_row_group_prepare lays out the template
// table (each call as at row 0) in host_table (gemm_group_bytes(capacity) bytes, copied to device memory by the
// caller) and the launch shape for at most max_tiles tiles; launch_gemm_row_group_fill writes the live table from the
// template and the starts before each launch_gemm_group. Each output is bit-identical to launch_gemm of its call.
struct GemmRowShift {
    int64_t a = 0, b = 0, c = 0, add = 0;  // elements each operand advances per grouped row
    int rows_in_reduction = 0;            // the row count is the reduction length (weight gradients), else I
};
int gemm_row_group_prepare(const GemmCall* calls, int n, int capacity, int tile, int64_t max_tiles, void* host_table,
                           GemmGroup* group);
int launch_gemm_row_group_fill(const void* device_templ, void* device_table, const GemmGroup& group,
                               const int64_t* device_start, const GemmRowShift& shift, hipStream_t stream);

// dst[r][c] = src[r][c] and dstT[c][r] = src[r][c] as doubles (either may be null).
int launch_to_double(const float* src, int64_t rows, int64_t cols, int64_t lds, double* dst, int64_t ldd,
                     double* dstT, int64_t lddT, hipStream_t stream);
int launch_transpose_f32(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t stream);
// dst = src^T for many matrices in one launch: transpose_batch_tiles fills the n + 1 tile starts (host) and returns
// the tile count; the jobs and the starts are then passed in device memory.
struct TransposeJob {
    const float* src;
    int64_t rows, cols;
    float* dst;
};
int64_t transpose_batch_tiles(const TransposeJob* jobs, int n, int64_t* tile_start);
int launch_transpose_batch(const TransposeJob* device_jobs, const int64_t* device_tile_start, int n, int64_t tiles,
                           hipStream_t stream);

// ---- row-local and elementwise kernels (rows.hip) ----

// rms_norm (nn.hpp:391-408); inv_rms (optional, double per row) records 1/sqrt(mean(x^2)+eps).
int launch_rms_norm(const float* x, const float* w, float* out, int64_t rows, int64_t dim, double eps, int unit_offset,
                    double* inv_rms, hipStream_t stream);
// rms_norm_backward's dx (grad.hpp:79-105): dx = addend + dx_norm when addend is given (the residual glue); writes
// inv_rms per row for the weight gradient.
int launch_rms_norm_backward_dx(const float* x, const float* w, const float* dy, float* dx, const float* addend,
                                int64_t rows, int64_t dim, double eps, int unit_offset, double* inv_rms,
                                hipStream_t stream);
// Column sums over segments of rows with a float sum over segments (rms_norm dw, linear db):
//   part[s][i] = f32(sum over rows r of segment s, ascending, of term(r, i))   then out[i] = window-ordered sum.
// kind 0: term = dy[r][i] (bias); kind 1: term = (dy[r][i] x[r][i]) inv_rms[r] (norm weight). weights (device,
// nseg floats, may be null): each segment's sum is multiplied by its factor before the window-ordered sum; colscale
// (device, dim floats, may be null): each segment's column i is first multiplied by colscale[i].
int launch_column_sums(int kind, const float* dy, const float* x, const double* inv_rms, int64_t dim,
                       const int64_t* seg_host, int nseg, float* partial, float* out, hipStream_t stream,
                       const float* weights = nullptr, const float* colscale = nullptr);
// rope (nn.hpp:501-530) with precomputed cos/sin tables [positions][half] (double, sin already negated for inverse).
int launch_rope_tables(const int64_t* positions, int64_t n, const double* inv_freq, int64_t half, double* cos_table,
                       double* sin_table, hipStream_t stream);
// rope (non-interleaved) of two tensors of the same tokens in one launch.
int launch_rope_pair(const float* x1, float* out1, int64_t heads1, const float* x2, float* out2, int64_t heads2,
                     const int64_t* pos_index, const double* cos_table, const double* sin_table, int64_t tokens,
                     int64_t head_dim, int64_t rotary_dim, int inverse, hipStream_t stream);
// rope without tables (cos and sin computed per token in the kernel); rows of at most 64 elements
int launch_rope_direct(const float* x, const int64_t* positions, const double* inv_freq, float* out, int64_t tokens,
                       int64_t heads, int64_t head_dim, int64_t rotary_dim, int interleaved, int inverse,
                       hipStream_t stream);
int launch_rope(const float* x, const int64_t* pos_index, const double* cos_table, const double* sin_table,
                float* out, int64_t tokens, int64_t heads, int64_t head_dim, int64_t rotary_dim, int interleaved,
                int inverse, hipStream_t stream);
int launch_silu(const float* x, float* out, int64_t n, hipStream_t stream);
// gate_act = silu(gate) (saved), product = gate_act * up (nn.hpp:489-492 and backprop.py:492-499); activation 1
// takes gelu_tanh instead of silu.
int launch_swiglu_forward(const float* gate, const float* up, float* gate_act, float* product, int64_t n,
                          hipStream_t stream, int activation = 0);
int launch_silu_backward(const float* x, const float* dy, float* out, int64_t n, hipStream_t stream);
// A device-to-device copy of `bytes` (16-byte vectors when both pointers allow).
int launch_device_copy(void* dst, const void* src, size_t bytes, hipStream_t stream);
// gelu_tanh elementwise (nn.hpp:481-485) and the gated form f32(gelu_tanh(gate)) * up (nn.hpp:488-492).
int launch_gelu_tanh(const float* x, float* out, int64_t n, hipStream_t stream);
int launch_geglu_tanh(const float* gate, const float* up, float* out, int64_t n, hipStream_t stream);
int launch_gelu_tanh_backward(const float* x, const float* dy, float* out, int64_t n, hipStream_t stream);
int launch_softcap_backward(const float* x, const float* dy, float* out, int64_t n, double cap, hipStream_t stream);
// softcap (nn.hpp:457-461): out = f32(cap tanh(x / cap)), in double
int launch_softcap(const float* x, float* out, int64_t n, double cap, hipStream_t stream);
// out = f32(sigmoid(x)) elementwise (nn.hpp:464)
int launch_sigmoid(const float* x, float* out, int64_t n, hipStream_t stream);
// _swiglu_backward's elementwise glue (backprop.py:301-303): dgate = silu_backward(gate, dproduct * up),
// dup = dproduct * gate_act.
int launch_swiglu_backward(const float* gate, const float* up, const float* gate_act, const float* dproduct,
                           float* dgate, float* dup, int64_t n, hipStream_t stream, int activation = 0);
int launch_add(const float* a, const float* b, float* out, int64_t n, hipStream_t stream);
// out[i] = window-ordered float sum over s of f32(partial[s][i] weights[s]) (weights null: 1)
int launch_segment_sums(const float* partial, int64_t dim, int nseg, const float* weights, float* out,
                        hipStream_t stream);
// The shared expert's gate (backprop.py:339-351, 519-524): forward s = f32(sigmoid(h2 w)), term = f32(y s) (w null:
// term = y); backward dy = f32(dmlp s), dscore = f32(f32(dot(dmlp, y) s) (1 - s)), then dh += f32(dscore w) (dh
// non-null) and part[window][k] = the window's f32(sum dscore h2[.][k]) (part non-null); with dy null, dscore is
// taken as already formed.
int launch_shared_gate_forward(const float* h2, const float* w, const float* y, float* s, float* term, int64_t rows,
                               int64_t H, hipStream_t stream);
int launch_shared_gate_backward(const float* dmlp, const float* y, const float* s, const float* w, const float* h2,
                                float* dy, float* dscore, float* dh, const int64_t* seg, int nseg, float* part,
                                int64_t rows, int64_t H, hipStream_t stream);
// x = f32(x * f), or f32(x / f) with divide, in place
int launch_scale(float* x, int64_t n, float f, bool divide, hipStream_t stream);
int launch_add3(const float* a, const float* b, const float* c, float* out, int64_t n, hipStream_t stream);
int launch_gather_rows(const float* table, const int64_t* index, float* out, int64_t rows, int64_t dim,
                       hipStream_t stream);

// ---- mixture of experts (moe.hip) ----

// moe_route (nn.hpp:864-896): indices/weights [rows][k] in rank order; probs [rows][experts] (optional) the softmax.
int launch_moe_route(const float* logits, int64_t rows, int64_t experts, int64_t k, int normalize, int64_t* indices,
                     float* weights, float* probs, hipStream_t stream);
// moe_route_backward (grad.hpp:507-541); dprob [rows][experts] may be null.
int launch_moe_route_backward(const float* logits, const int64_t* indices, const float* dweights, const float* dprob,
                              int64_t rows, int64_t experts, int64_t k, int normalize, float* dlogits,
                              hipStream_t stream);
// out[r] = (0 + the row's k terms in expert order) + addend[r] (addend may be null: no addition); term =
// y[order] * weights[slot] or y[order].
int launch_moe_combine(const float* y, const int64_t* order, const int64_t* slot, const float* weights,
                       const float* addend, float* out, int64_t rows, int64_t k, int64_t dim, hipStream_t stream);
// dweights[slot[p]] = dot(dout[row_of[p]], y[p]) and dy[p] = dout[row_of[p]] * weights[slot[p]] per position p.
int launch_moe_dweights(const float* dout, const float* y, const int64_t* row_of, const int64_t* slot,
                        const float* weights, int64_t positions, int64_t dim, float* dweights, float* dy,
                        hipStream_t stream);
// Groups the rows of one routed layer by expert on the device (experts ascending, rows ascending in each expert:
// np.nonzero's order): estart [E + 1] the group starts, eseg [E][eseg_ld] each group's window boundaries (nseg + 1
// used), row_of / slot [rows K] the row and choice of each grouped position, order [rows K] each row's positions by
// ascending expert, pos_of [rows K] scratch, counts [nseg][E] += the layer's choices per window (router
// statistics), err set to 1 for an expert out of range; cnt_scratch holds nseg E 8-byte counters.
int launch_moe_group_rows(const int64_t* chosen, int64_t rows, int64_t K, int64_t E, const int64_t* seg, int nseg,
                          void* cnt_scratch, int64_t* estart, int64_t* eseg, int64_t eseg_ld, int64_t* row_of,
                          int64_t* slot, int64_t* order, int64_t* pos_of, int64_t* counts, int* err,
                          hipStream_t stream);
int launch_zero_i64(int64_t* x, int64_t n, hipStream_t stream);
// The router load-balancing loss per window (backprop.py:359-377); grad_row [nseg][experts] may be null.
int launch_router_stats(const float* probs, int64_t layer_stride, int64_t layers, const int64_t* seg, int nseg,
                        const int64_t* counts, int64_t experts, double router_scale, double* loss, float* grad_row,
                        hipStream_t stream);
// softmax of each row (math.hpp:387-398), column_mean (interp.hpp:146-155), dot (math.hpp:31-37: one serial chain;
// result is a device float).
int launch_softmax_rows(const float* logits, float* out, int64_t rows, int64_t n, hipStream_t stream);
int launch_column_mean(const float* x, float* out, int64_t rows, int64_t cols, hipStream_t stream);
int launch_dot(const float* a, const float* b, int64_t n, float* result, hipStream_t stream);
int launch_broadcast_window_rows(const float* grad_row, const int64_t* seg, int nseg, int64_t rows, int64_t experts,
                                 float* out, hipStream_t stream);

// ---- attention (attention.hip) ----

struct AttentionShape {
    int64_t q_len, kv_len;  // packed totals over all sequences
    int64_t q_heads, kv_heads, head_dim, value_dim;
    double scale;
    int causal;
    int64_t q_offset, window;
    double softcap;
};

// Segments: `count` independent sequences; sequence s has queries [q_off[s], q_off[s] + q_len[s]) and keys
// [kv_off[s], ...) of the packed tensors (device arrays). A plain call is one sequence.
struct AttentionBatch {
    const int64_t* q_start;   // device [count]
    const int64_t* q_len;     // device [count]
    const int64_t* kv_start;  // device [count]
    const int64_t* kv_len;    // device [count]
    int count;
    int64_t max_q, max_kv;    // host bounds of the lengths
};

// Rows (query, head) whose keys do not fit the kernels' LDS staging (more than 2048) stage them in device memory:
// `stage` holds attention_stage_bytes (0 when every row fits in LDS).
size_t attention_stage_bytes(const AttentionShape& s, const AttentionBatch& b, bool backward);
int launch_attention(const float* q, const float* k, const float* v, float* out, const AttentionShape& s,
                     const AttentionBatch& b, void* stage, hipStream_t stream);
// Workspace bytes of attention_backward: the probabilities and score gradients of every row.
size_t attention_backward_workspace(const AttentionShape& s, const AttentionBatch& b, int64_t total_q);
int launch_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                              float* dv, const AttentionShape& s, const AttentionBatch& b, int64_t total_q,
                              int64_t total_kv, void* workspace, void* stage, hipStream_t stream);

// ---- self-attention on the matrix-core tiles (attn_abi.hip) ----
// One sequence with q_len == kv_len = n, q_offset 0 (or negative), no soft-cap, head_dim == value_dim (a multiple
// of 4), causal with an optional sliding window or every key visible: the training step's attention path.
bool self_attention_fast(size_t q_len, size_t kv_len, size_t q_heads, size_t kv_heads, size_t head_dim,
                         size_t value_dim, int causal, int64_t q_offset, size_t window, double softcap);
size_t self_attention_workspace(size_t n, size_t q_heads, size_t kv_heads, size_t head_dim, bool backward);
int self_attention_forward(const float* q, const float* k, const float* v, float* out, size_t n, size_t q_heads,
                           size_t kv_heads, size_t head_dim, double scale, int causal, int64_t window, void* ws,
                           hipStream_t s);
int self_attention_backward(const float* q, const float* k, const float* v, const float* dout, float* dq, float* dk,
                            float* dv, size_t n, size_t q_heads, size_t kv_heads, size_t head_dim, double scale,
                            int causal, int64_t window, void* ws, hipStream_t s);

// ---- loss and embedding (loss.hip) ----

// cross_entropy (grad.hpp:395-426) over segments: per row the dlogits, and the summed loss of each segment
// (rows ascending, double) into loss_out[s] (seg_dev: nseg + 1 row offsets in device memory). row_max, row_total,
// row_loss: workspace of rows doubles each. error_flag is set to 1 when a target is >= vocab.
int launch_cross_entropy(const float* logits, const int64_t* targets, float* dlogits, int64_t rows, int64_t vocab,
                         double scale, const int64_t* seg_dev, int nseg, double* row_max, double* row_total,
                         double* row_loss, double* loss_out, int* error_flag, hipStream_t stream);
// out[v] = sum over rows with tokens == v, in row order (grad.hpp:431-464), from a host-built grouping:
// group g covers order[start[g] .. start[g+1]) and writes row out_row[g].
int launch_embedding_groups(const float* dy, int64_t dim, const int64_t* order, const int64_t* start,
                            const int64_t* out_row, int64_t groups, float* out, int64_t ld_out, hipStream_t stream);

// ---- optimizer (optim.hip) ----

// Serial sum of squares of each tensor (grad.hpp:467-473), tensors given by device arrays of (offset, count) into
// one arena; then the total over tensors in table order, its square root and the clipping scale
// (optimizer.py:66-90), all in double on the device: stats = {total, norm, clip}.
int launch_global_norm(const float* arena, const int64_t* offsets, const int64_t* counts, int64_t tensors,
                       double* per_tensor, double max_grad_norm, double* stats, hipStream_t stream);
int launch_sum_squares(const float* values, int64_t n, double* result, hipStream_t stream);
// total = sum of per_tensor in order, norm = sqrt(total), clip factor (optimizer.py:66-90): stats = {total, norm, clip}.
int launch_norm_finish(const double* per_tensor, int64_t tensors, double max_grad_norm, double* stats,
                       hipStream_t stream);

// ---- exact parallel sum of squares (sumsq.hip) ----
// Tensors of one arena split into fixed blocks of kSumSquaresBlock values; the plan arrays live in device memory.
constexpr int64_t kSumSquaresBlock = 8192;
struct ExactSumPlan {
    int64_t tensors = 0, blocks = 0;
    const int64_t* tfirst = nullptr;   // [tensors] first block of each tensor
    const int64_t* tblocks = nullptr;  // [tensors] block count of each tensor
    const int64_t* bstart = nullptr;   // [blocks] arena offset of each block
    const int64_t* bcount = nullptr;   // [blocks] elements in each block
};
size_t exact_sum_squares_blocks(const int64_t* counts, int64_t tensors);
void exact_sum_squares_plan(const int64_t* offsets, const int64_t* counts, int64_t tensors, int64_t* tfirst,
                            int64_t* tblocks, int64_t* bstart, int64_t* bcount);
size_t exact_sum_squares_workspace(size_t blocks);
// per_tensor[t] = the serial double sum of squares of tensor t, bit for bit (grad.hpp:467-473).
int launch_exact_sum_squares(const float* arena, const ExactSumPlan& plan, void* workspace, double* per_tensor,
                             hipStream_t stream);
// adamw_step (grad.hpp:481-495) over an arena; chunk table: chunk c covers [chunk_start[c], chunk_end[c]) with
// weight decay chunk_decay[c]; grad_scale read from device memory (the clip factor) when grad_scale_dev != null.
struct AdamWArgs {
    double lr, beta1, beta2, eps, bc1, bc2, grad_scale;
};
int launch_adamw_plain(float* param, const float* grad, float* m, float* v, int64_t n, double weight_decay,
                       const AdamWArgs& a, hipStream_t stream);
int launch_adamw(float* param, const float* grad, float* m, float* v, const int64_t* chunk_start,
                 const int64_t* chunk_end, const double* chunk_decay, int64_t chunks, const AdamWArgs& a,
                 const double* grad_scale_dev, hipStream_t stream);

// ---- LoRA and the Q8_0 base (lora.hip) ----

int launch_quantize_q8_0(const float* x, int8_t* q, float* scales, int64_t n, hipStream_t stream);
// out[r][n] = linear_q8 of the quantised activations (xq int8 [rows][K], xs [rows][K / 32]) and weights (wq [N][K],
// ws [N][K / 32]) (quant.hpp:143-169): exact int32 block dots on the int8 matrix cores, combined in double.
int launch_linear_q8(const int8_t* xq, const float* xs, const int8_t* wq, const float* ws, const float* bias,
                     float* out, int64_t rows, int64_t K, int64_t N, hipStream_t stream);
int launch_dequantize_q8_0(const int8_t* q, const float* scales, float* out, int64_t n, hipStream_t stream);
// out = base + x * s in float32 (base may be null: out = x * s)
int launch_scale_add(const float* base, const float* x, float s, float* out, int64_t n, hipStream_t stream);
// out = weight + f32(linear(b, a^T)) * scale; a [rank][in], b [out][rank] (lora.py:271-276)
size_t lora_merge_workspace(int64_t out_f, int64_t in_f, int64_t rank);
int launch_lora_merge(const float* weight, const float* a, const float* b, float* out, int64_t out_f, int64_t in_f,
                      int64_t rank, float scale, void* ws, size_t ws_bytes, hipStream_t stream);
// da = f32(linear(b^T, grad^T)) * scale, db = f32(linear(grad, a)) * scale (lora.py:374-383)
size_t lora_adapter_gradients_workspace(int64_t out_f, int64_t in_f, int64_t rank);
int launch_lora_adapter_gradients(const float* grad, const float* a, const float* b, float* da, float* db,
                                  int64_t out_f, int64_t in_f, int64_t rank, float scale, void* ws, size_t ws_bytes,
                                  hipStream_t stream);

}  // namespace dllm_hip
