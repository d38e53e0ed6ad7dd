/*
 * attn_mi355x.h -- C ABI of the MI355X (gfx950) attention hot path.
 *
 * Drop-in replacement for the attention launch API of MarcVivas/llm-inference
 * (include/kernels/kernels.hpp).  Each entry point names the reference
 * declaration it replaces.  All device buffers are caller-owned; no entry
 * point allocates, frees or copies host<->device, so every launch is safe to
 * record into a HIP graph.  fp16 buffers are IEEE binary16 (attn_f16_t holds
 * the bit pattern).  Strides are in elements between consecutive tokens; a
 * stride of 0 means "packed" (causal_attention.hip.cpp:412-413, :875-876).
 *
 * Return value: 0 (hipSuccess) or a hipError_t code.  Shapes the reference
 * launchers silently ignore (seq_len == 0, kv_len == 0, num_kv_heads == 0,
 * num_heads % num_kv_heads != 0; causal_attention.hip.cpp:392-399, :860-866,
 * :945-946; rope.hip.cpp:156) return 0 and launch nothing, leaving every
 * output untouched.
 */
#ifndef ATTN_MI355X_H
#define ATTN_MI355X_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t attn_f16_t;

/* Decode workspace sizing unit: callers provide num_heads * ceil(kv_len /
 * ATTN_KV_CHUNK) partial states (kernels.hpp:103 `#define KV_CHUNK 12`). */
#define ATTN_KV_CHUNK 12

/* Fused RoPE + KV-cache append.
 * Replaces launch_rope_and_store_kv (kernels.hpp:62-79; rope.hip.cpp:138-196).
 * Token t: Q heads rotated in place at q + t*q_stride + h*D; K rotated into
 * k_cache row (start_pos + t) (K source unchanged) and V copied to v_cache row
 * (start_pos + t); cache rows are num_kv_heads*head_dim elements apart.
 * apply_rotation == 0 (NoPE layers): K and V copied, Q untouched.
 * k_cache == NULL: K rotated in place, V untouched (the launch_rope mode).
 * V is read with k_stride.  cos/sin tables are [max_seq_len][head_dim/2]. */
int attn_rope_store_kv(attn_f16_t* q, attn_f16_t* k, const attn_f16_t* v,
                       attn_f16_t* k_cache, attn_f16_t* v_cache,
                       const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                       size_t seq_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                       size_t q_stride, size_t k_stride, size_t start_pos,
                       int apply_rotation, hipStream_t stream);

/* In-place RoPE of Q and K.
 * Replaces launch_rope (kernels.hpp:47-59; rope.hip.cpp:198-205).  The
 * reference launches on the null stream; pass NULL for identical behaviour. */
int attn_rope(attn_f16_t* q, attn_f16_t* k, const attn_f16_t* cos_table,
              const attn_f16_t* sin_table, size_t seq_len, size_t num_heads,
              size_t num_kv_heads, size_t head_dim, size_t q_stride, size_t k_stride,
              size_t start_pos, hipStream_t stream);

/* Re-point a captured RoPE/append node at a new position.
 * Replaces update_rope_and_store_kv_node (kernels.hpp:81-86;
 * rope.hip.cpp:208-241). */
int attn_update_rope_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t start_pos,
                          int apply_rotation);

/* Causal GQA prefill: query t of head h attends to keys 0..t of KV head
 * h / (num_heads/num_kv_heads); output packed [seq_len][num_heads][head_dim].
 * Replaces launch_causal_attention_prefill (kernels.hpp:88-99;
 * causal_attention.hip.cpp:376-451), which launches on the null stream: pass
 * NULL for identical behaviour. */
int attn_prefill(const attn_f16_t* q, const attn_f16_t* k, const attn_f16_t* v,
                 attn_f16_t* out, size_t seq_len, size_t num_heads, size_t num_kv_heads,
                 size_t head_dim, size_t q_stride, size_t kv_stride, hipStream_t stream);

/* Flash-Decode of one query token over kv_len cached keys (no mask: all
 * kv_len keys are visible).  q is read packed [num_heads][head_dim] (q_stride
 * and start_pos are accepted and unused, as in the reference); out is packed
 * [num_heads][head_dim].  partial_out/max/sum are caller-owned workspace of at
 * least num_heads*ceil(kv_len/ATTN_KV_CHUNK) states (partial_out: x head_dim
 * floats); their contents are private to this library and nothing past that
 * capacity is written.  For head_dim 128 two kernels are enqueued, the split
 * kernel (*attention_node) and the partial merge (*merge_node), as in the
 * reference; up to 384 keys the split kernel alone when merge_node is NULL
 * (one workgroup per KV head writes the output; with merge_node the merge
 * kernel follows and exits at once, so that an updater can move the pair to
 * a longer context); other shapes enqueue one generic kernel and both
 * handles receive it.
 * Replaces launch_causal_attention_decode (kernels.hpp:104-123) and
 * launch_causal_attention_decode_vectorized (kernels.hpp:127-146;
 * causal_attention.hip.cpp:840-972). */
int attn_decode(const attn_f16_t* q, const attn_f16_t* k_cache, const attn_f16_t* v_cache,
                attn_f16_t* out, float* partial_out, float* partial_max, float* partial_sum,
                size_t query_len, size_t kv_len, size_t start_pos, size_t num_heads,
                size_t num_kv_heads, size_t head_dim, size_t q_stride, size_t kv_stride,
                hipStream_t stream, hipGraphNode_t* attention_node, hipGraphNode_t* merge_node);

/* Re-point a captured decode node at a new kv_len (split plan, grid and the
 * split kernel's heads-per-workgroup variant are recomputed, as a launch at
 * that kv_len would choose them).  Replaces update_causal_attention_decode_node
 * (kernels.hpp:190-194; causal_attention.hip.cpp:975-1001). */
int attn_update_decode_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t kv_len);

/* Re-point a captured merge node at a new kv_len (its split count).  For the
 * single-kernel generic path this is a no-op.  Replaces
 * update_merge_attention_decode_node (kernels.hpp:148-152;
 * causal_attention.hip.cpp:1003-1026). */
int attn_update_merge_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t kv_len);

/* Node records (no counterpart in the reference; a diagnostic).  Every kernel
 * this library launches while its stream is capturing is recorded, with its
 * launch configuration and argument as captured, until the graph holding it
 * is released (a user object retained by that graph drops its records).  The
 * attn_update_* functions patch a recorded node from its record; the
 * reference updaters read every node back with hipGraphKernelNodeGetParams
 * (causal_attention.hip.cpp:981,1009; rope.hip.cpp:215), which is what is
 * done here for nodes without a record.  Returns the number of records
 * held. */
size_t attn_graph_node_records(void);

/* No single counterpart in the reference: launch_rope_and_store_kv(q, k, v,
 * k_cache, v_cache, cos, sin, 1, Hq, Hkv, D, 0, 0, start_pos,
 * apply_rotation) followed by launch_causal_attention_decode(q, k_cache,
 * v_cache, out, partials, 1, kv_len, start_pos, Hq, Hkv, D, 0, kv_stride,
 * stream, ...) -- the pair ModelInference issues per layer in every decode
 * step (model_inference.hpp:96-126) -- as the decode's two kernels: the split
 * kernel rotates q in registers and appends the new K (rotated) / V row
 * before reading it, the merge kernel leaves q rotated in place.  q, the
 * cache and out equal that pair's bit for bit.  Serves the MFMA decode path
 * (head_dim 128, 16-byte aligned tensors) with kv_stride = Hkv*D (or 0) and
 * start_pos < kv_len.  Other shapes called without node handles issue the
 * pair itself (attn_rope_store_kv, then attn_decode); with node handles
 * requested they return hipErrorInvalidValue and enqueue nothing, since
 * attn_update_rope_decode_nodes patches only the fused pair.  The node
 * handles are the split and merge kernels, patched together by
 * attn_update_rope_decode_nodes. */
int attn_rope_store_kv_decode(attn_f16_t* q, const attn_f16_t* k, const attn_f16_t* v,
                              attn_f16_t* k_cache, attn_f16_t* v_cache,
                              const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                              attn_f16_t* out, float* partial_out, float* partial_max,
                              float* partial_sum, size_t kv_len, size_t start_pos,
                              size_t num_heads, size_t num_kv_heads, size_t head_dim,
                              size_t kv_stride, int apply_rotation, hipStream_t stream,
                              hipGraphNode_t* attention_node, hipGraphNode_t* merge_node);

/* Patches both captured nodes of attn_rope_store_kv_decode to a new kv_len,
 * start_pos and apply_rotation (what update_rope_and_store_kv_node,
 * update_causal_attention_decode_node and update_merge_attention_decode_node
 * do for the separate launches). */
int attn_update_rope_decode_nodes(hipGraphExec_t graph_exec, hipGraphNode_t attention_node,
                                  hipGraphNode_t merge_node, size_t kv_len, size_t start_pos,
                                  int apply_rotation);

/* No counterpart in the reference: attn_decode (query_len 1, start_pos and
 * q_stride unused) without a caller workspace, for callers that cannot
 * allocate device memory (code under graph capture that must not call
 * hipMalloc, tight serving loops, harnesses that forbid it).  Same plan,
 * kernels and output bits as attn_decode; the partial states go to a
 * library-owned array of ATTN_DECODE_NOALLOC_SCRATCH_BYTES per GPU (held
 * until the process ends; its address is looked up once per device on the
 * first call there).  A plan whose states exceed the array (more than
 * ATTN_DECODE_NOALLOC_SCRATCH_BYTES / 264 query-head x split states; every
 * SmolLM3 decode shape uses at most 2048) returns hipErrorInvalidValue and
 * enqueues nothing.  Allocates nothing; not for graph capture of node handles
 * (none are returned).  Every call on one GPU shares the array: calls that
 * overlap on one GPU (unordered streams) race and must not be issued. */
#define ATTN_DECODE_NOALLOC_SCRATCH_BYTES (2u << 20)
int attn_decode_noalloc(const attn_f16_t* q, const attn_f16_t* k_cache,
                        const attn_f16_t* v_cache, attn_f16_t* out, size_t kv_len,
                        size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t kv_stride,
                        hipStream_t stream);

/* Workspace states a caller must provide for kv_len keys:
 * num_heads * ceil(kv_len / ATTN_KV_CHUNK) (model_inference.hpp:192-198). */
size_t attn_decode_workspace_states(size_t num_heads, size_t kv_len);

/* launch_qkv_decode (kernels.hpp:38-45; qkv_gemm.hip.cpp:107-116, the GEMV of
 * matrix_vec_mul.hip.cpp:79-172 with beta = 0): y[total_qkv_dim] =
 * W[total_qkv_dim][hidden_size] x[hidden_size], fp16 in, fp32 accumulation,
 * fp16 out; W row-major with the Q rows of all heads, then K, then V.
 * total_qkv_dim == 0 is a no-op; hidden_size == 0 writes zeros (x, W may then
 * be null).  Any length and alignment (16-byte loads when hidden_size % 8 == 0
 * and x, W are 16-byte aligned, element loads otherwise). */
int attn_qkv_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w, size_t hidden_size,
                    size_t total_qkv_dim, hipStream_t stream);

/* No single counterpart in the reference: launch_qkv_decode followed by
 * launch_rope_and_store_kv(y, y + Hq*D, y + (Hq+Hkv)*D, k_cache, v_cache, cos,
 * sin, 1, Hq, Hkv, D, total, total, start_pos, apply_rotation) -- the pair
 * ModelInference issues back to back in every decode step
 * (model_inference.hpp:354-369) -- as one kernel.  Results equal that pair's
 * bit for bit.  For callers that control the decode step (one fewer graph node
 * and no round trip of Q and K through memory). */
int attn_qkv_rope_store_kv_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                                  attn_f16_t* k_cache, attn_f16_t* v_cache,
                                  const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                                  size_t hidden_size, size_t num_heads, size_t num_kv_heads,
                                  size_t head_dim, size_t start_pos, int apply_rotation,
                                  hipStream_t stream);

/* Patches start_pos / apply_rotation of a captured
 * attn_qkv_rope_store_kv_decode node (as update_rope_and_store_kv_node does for
 * the RoPE node, rope.hip.cpp:208-241). */
int attn_update_qkv_rope_node(hipGraphExec_t graph_exec, hipGraphNode_t node, size_t start_pos,
                              int apply_rotation);

/* launch_attention_out_projection_decode (kernels.hpp:179-187;
 * attention_out_projection.hip.cpp:61-71, the GEMV of
 * matrix_vec_mul.hip.cpp:79-172): y[hidden_size] = W[hidden_size][num_heads *
 * head_dim] x + beta * y, fp16 in, fp32 accumulation (beta * y added to the
 * fp32 sum when beta != 0), fp16 out.  hidden_size == 0 is a no-op; an empty
 * row (num_heads * head_dim == 0) leaves beta * y.  The engine calls it with
 * beta = 1 on the residual stream (model_inference.hpp:390-397). */
int attn_out_proj_decode(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                         size_t hidden_size, size_t num_heads, size_t head_dim, float beta,
                         hipStream_t stream);

/* No single counterpart in the reference: launch_causal_attention_decode(q,
 * k_cache, v_cache, attn_out, partials, 1, kv_len, kv_len - 1, Hq, Hkv, D, 0,
 * kv_stride, ...) followed by launch_attention_out_projection_decode(attn_out,
 * y, w_o, hidden_size, Hq, D, beta) -- the pair ModelInference issues per layer
 * in every decode step (model_inference.hpp:371-397).  By default it issues
 * exactly those two launches (split + merge kernels, then the o_proj GEMV).
 * With attn_set_option("decode_out_proj_fused", 1), decode shapes on the MFMA
 * path (head_dim 128) run the split kernel (*attention_node) and one kernel
 * that merges each head's partial states and multiplies the result by W_o
 * (*merge_node); attn_out still receives the attention output, and y matches
 * the pair within fp32 rounding of the partial sums (heads summed in order;
 * deterministic).  The fused form is measured slower on MI355X (its cross-XCD
 * reduction of the heads costs more than the kernel boundary it removes) and
 * stays selectable for that measurement; it splits every context (no
 * one-kernel decode of short contexts, see "decode_whole_max_keys").  Other
 * shapes, or a null workspace, always issue the two launches.
 * out_proj_workspace:
 * attn_decode_out_proj_workspace_bytes(Hq, hidden_size) bytes, 256-byte
 * aligned, ZERO-FILLED once before the first call; every call leaves its
 * counters zero again.  Calls sharing a workspace must be ordered (one
 * stream); update_merge/attn_update_merge_node patches the fused node like
 * the merge node. */
size_t attn_decode_out_proj_workspace_bytes(size_t num_heads, size_t hidden_size);
int attn_decode_out_proj(const attn_f16_t* q, const attn_f16_t* k_cache, const attn_f16_t* v_cache,
                         attn_f16_t* attn_out, float* partial_out, float* partial_max,
                         float* partial_sum, size_t kv_len, size_t num_heads,
                         size_t num_kv_heads, size_t head_dim, size_t kv_stride,
                         const attn_f16_t* w_o, attn_f16_t* y, size_t hidden_size, float beta,
                         void* out_proj_workspace, hipStream_t stream,
                         hipGraphNode_t* attention_node, hipGraphNode_t* merge_node);

/* launch_qkv_gemm (kernels.hpp:29-36; qkv_gemm.hip.cpp:7-105, a rocBLAS
 * gemm_ex with fp32 compute): y[seq_len][total_qkv_dim] =
 * x[seq_len][hidden_size] . W[total_qkv_dim][hidden_size]^T, fp16 in, fp32
 * accumulation, fp16 out, all row-major and packed.  seq_len == 0 or
 * total_qkv_dim == 0 is a no-op; hidden_size == 0 writes zeros (x, W may then
 * be null).  fp16 MFMA when hidden_size % 64 == 0 and x, W are 16-byte
 * aligned; any other shape runs a plain fp32-accumulating kernel. */
int attn_qkv_gemm(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w, size_t seq_len,
                  size_t hidden_size, size_t total_qkv_dim, hipStream_t stream);

/* No single counterpart in the reference: launch_qkv_gemm followed by
 * launch_rope_and_store_kv(y, y + Hq*D, y + (Hq+Hkv)*D, k_cache, v_cache, cos,
 * sin, seq_len, Hq, Hkv, D, total, total, start_pos, apply_rotation) -- the
 * pair ModelInference issues back to back in prefill (model_inference.hpp:
 * 266-285) -- as one kernel when head_dim == 128, the GEMM takes its MFMA
 * path and y, the caches and the tables are 16-byte aligned (the two launches
 * otherwise).  Results equal attn_qkv_gemm followed by
 * attn_rope_store_kv bit for bit. */
int attn_qkv_gemm_rope_store_kv(const attn_f16_t* x, attn_f16_t* y, const attn_f16_t* w,
                                attn_f16_t* k_cache, attn_f16_t* v_cache,
                                const attn_f16_t* cos_table, const attn_f16_t* sin_table,
                                size_t seq_len, size_t hidden_size, size_t num_heads,
                                size_t num_kv_heads, size_t head_dim, size_t start_pos,
                                int apply_rotation, hipStream_t stream);

/* Host-side RoPE tables, fp16 [max_seq_len][head_dim/2]: inv_freq[i] =
 * 1/powf(theta, 2i/D), angle = float(pos)*inv_freq[i], cos/sin in fp32 then
 * RNE to fp16.  Same tables as rope_cache.hpp:48-76 (create_rope_cache minus
 * the upload).  Pure host code. */
int attn_rope_tables(attn_f16_t* cos_out, attn_f16_t* sin_out, size_t max_seq_len,
                     size_t head_dim, float rope_theta);

/* ---- weights.bin: the model file the engine maps (python/export_weights.py;
 * include/model_config.hpp, model.hpp:18-93, device_weights.hpp:57-110).
 * Layout: the 44-byte header below; uint32 tokenizer-JSON length; the JSON;
 * zero padding to a 64-byte file offset; then fp16 tensors back to back:
 * embedding [vocab][hidden]; per layer input_norm [hidden], q_proj
 * [Hq*D][hidden], k_proj [Hkv*D][hidden], v_proj [Hkv*D][hidden], (q_norm [D],
 * k_norm [D] only if the checkpoint has them), o_proj [hidden][Hq*D],
 * post_attention_norm [hidden], gate_proj, up_proj [inter][hidden], down_proj
 * [hidden][inter]; final norm [hidden]; lm_head [vocab][hidden].  q_proj, k_proj
 * and v_proj are adjacent, so q_proj is the fused [Hq*D + 2*Hkv*D][hidden] QKV
 * weight the projections above take.  Pure host code (no HIP calls). */
typedef struct attn_model_config {   /* model_config.hpp:10-24, 44 bytes */
    char magic[4];                   /* "QWEN" */
    uint32_t vocab_size, hidden_size, num_layers, num_heads, num_kv_heads, head_dim,
        intermediate_size, max_seq_len;
    float rms_norm_eps, rope_theta;
} attn_model_config;

/* Tensor offsets are in fp16 elements from the start of the weight payload;
 * layer l's tensors start at layer_base + l * layer_elems + the per-layer
 * offset.  q_norm / k_norm are UINT64_MAX when the file has none. */
typedef struct attn_weights_layout {
    attn_model_config config;
    uint32_t has_qk_norm;
    uint64_t tokenizer_offset, tokenizer_bytes;   /* JSON, file offset and length */
    uint64_t weights_offset;     /* file offset of the payload (multiple of 64) */
    uint64_t weights_bytes;      /* payload bytes present in the file */
    uint64_t layout_bytes;       /* payload bytes the tensors occupy (<= weights_bytes) */
    uint64_t embedding, final_norm, lm_head, layer_base, layer_elems;
    uint64_t input_norm, q_proj, k_proj, v_proj, q_norm, k_norm, o_proj, post_attn_norm,
        gate_proj, up_proj, down_proj;
} attn_weights_layout;

/* Format errors (negative; the messages are attn_weights_error_string's). */
#define ATTN_WEIGHTS_SHORT_HEADER        (-1) /* model_config.hpp:34-35 */
#define ATTN_WEIGHTS_BAD_MAGIC           (-2) /* model_config.hpp:39-40 */
#define ATTN_WEIGHTS_NO_TOKENIZER_LENGTH (-3) /* model.hpp:50-52 */
#define ATTN_WEIGHTS_TOKENIZER_TRUNCATED (-4) /* model.hpp:57-59 */
#define ATTN_WEIGHTS_NO_PAYLOAD          (-5) /* model.hpp:84-86 */
#define ATTN_WEIGHTS_PAYLOAD_SHORT       (-6) /* not checked by the reference */
#define ATTN_WEIGHTS_SIZE_OVERFLOW       (-7) /* not checked by the reference */

/* Parses a weights.bin of file_bytes bytes from its first head_bytes bytes
 * (at least min(file_bytes, 48): the header and the tokenizer length; the
 * JSON itself is not read), in the reference's order of checks
 * (model_config.hpp:33-43, model.hpp:40-93), then lays out the payload as
 * attn_weights_layout_for does.  Returns 0, a negative ATTN_WEIGHTS_* code, or
 * hipErrorInvalidValue for null pointers or a short head. */
int attn_weights_parse(const void* head, size_t head_bytes, uint64_t file_bytes,
                       attn_weights_layout* out);

/* Tensor layout of a payload of payload_bytes bytes for config (the claims of
 * device_weights.hpp:80-109, in the exporter's order export_weights.py:89-134).
 * Deviations, both for files the reference would read out of bounds or
 * misread: a payload smaller than the tensors is rejected
 * (ATTN_WEIGHTS_PAYLOAD_SHORT), and a payload of exactly the size with
 * q_norm/k_norm per layer (export_weights.py:108-111) lays them out after
 * v_proj (has_qk_norm = 1).  tokenizer_* and weights_offset are left 0. */
int attn_weights_layout_for(const attn_model_config* config, uint64_t payload_bytes,
                            attn_weights_layout* out);

/* Static message for an ATTN_WEIGHTS_* code (the reference's exception texts
 * where it has one), or NULL for an unknown code. */
const char* attn_weights_error_string(int code);

/* Introspection for tests and benchmarks: the decode plan chosen for a shape
 * on the current device.  out[0] = path (0 generic; 1, 2, 3 = MFMA split
 * kernel serving 4, 2, 1 KV heads per workgroup), out[1] = splits of the
 * context, out[2] = keys per split, out[3] = threads per workgroup, out[4] =
 * partial states per query head written to the workspace (at most
 * ceil(kv_len / ATTN_KV_CHUNK)). */
int attn_decode_plan(size_t kv_len, size_t num_heads, size_t num_kv_heads, size_t head_dim,
                     size_t kv_stride, const void* q, const void* k_cache,
                     const void* v_cache, uint32_t out[5]);

/* Prefill path chosen for a shape: 0 generic, 1 MFMA. */
int attn_prefill_plan(const void* q, const void* k, const void* v, const void* out,
                      size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t q_stride,
                      size_t kv_stride);

/* Process-wide switches for tests and benchmarks (not needed in production):
 * "decode_force_generic", "decode_splits" (0 = automatic),
 * "decode_heads_per_workgroup" (0 = automatic: 1 up to 12288 keys, 2 above
 * when Hkv is even; 1, 2 or 4 KV heads per split workgroup, reduced to what
 * Hkv allows), "decode_kdma" (0 = automatic: from 4096 keys with more than
 * 64 keys per split, and for the one-workgroup-per-head plans, the split
 * kernel reads K in whole 256-byte rows through LDS-DMA, otherwise straight
 * into registers; 1 = registers, 2 = LDS-DMA), "prefill_force_generic",
 * "qkv_gemm_force_generic", "qkv_gemm_tokens_per_wave" (0 = automatic; 32, 64
 * or 128 tokens per wave of the 256 x 128-tile MFMA GEMM), "qkv_gemm_wide"
 * (0 = automatic, from 7168 tokens; 1 = never; 2 = whenever N is a multiple
 * of 384 and Y is 16-byte aligned), "prefill_waves" (0 = automatic: 4-wave
 * workgroups of 32 queries up to 6144 tokens, 8-wave workgroups of 64 queries
 * above; 4 or 8 forces one), "prefill_stage_all" (0 = automatic: up to 256
 * tokens every key tile of a 4-wave workgroup is copied into LDS at once;
 * 1 = never), "prefill_split_keys" (0 = automatic: up to 1024 tokens one
 * workgroup per head and 32-query tile, its keys split over the waves and
 * combined through LDS, as 8 waves of 32 keys up to 32 tokens, 4 waves of
 * 64-key tiles up to 256 and 4 waves each streaming every 4th 32-key unit
 * above; 1 = never, also no key halves; 2 = 4 waves of 64-key tiles (up to
 * 256 tokens); 3 = 8 waves of 32 keys (up to 256 tokens); 4 = the
 * streaming form at any length), "prefill_key_halves" (0 = automatic: from
 * 1025 to 4096 tokens, unless "prefill_waves" or "prefill_split_keys" is
 * set, 8-wave workgroups of 32 queries x 4 heads whose two 4-wave groups
 * take the even and the odd key tiles and combine through LDS; 1 = never;
 * 2 = at any length), "decode_out_proj_fused" (see attn_decode_out_proj),
 * "graph_node_records" (0 = the updaters use node records; 1 = they read
 * every node back, as the reference does), "decode_whole_max_keys" (0 =
 * automatic: contexts up to 384 keys are decoded by one workgroup per KV
 * head whose fold writes the output, so attn_decode enqueues one kernel
 * unless the merge node is asked for, and that merge kernel then exits at
 * once; < 0 = never; > 0 = the longest such context).
 * Returns 0 or -1 for an unknown name. */
int attn_set_option(const char* name, long value);

/* Library build identification (static string). */
const char* attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ATTN_MI355X_H */
