/*
 * klc_moe.h — C ABI of the MI355X (gfx950) MoE expert path.
 *
 * The reference (KLCquant) is pure Python on PyTorch: its "interface" for this
 * path is the Python API of mxfp4_expert.py and streamed_moe_router.py, and
 * there is no FFI.  Each entry point below replaces the torch-eager code at
 * the cited reference lines; the Python package `klcquant_amd` (mxfp4_expert.py,
 * streamed_moe_router.py) binds these through ctypes and keeps the reference's
 * Python signatures.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise.
 *   - bfloat16 data is passed as 16-bit patterns (uint16_t), float32 as float.
 *   - Nothing here allocates device memory: outputs and scratch are passed in.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *     is asynchronous; calls are stream-ordered and thread-safe (state is per
 *     call, the error message is per calling thread).
 *   - Return value: KLC_OK (0) or a negative KLC_ERR_* code; klc_last_error()
 *     then describes the failure.  Argument checks happen before any launch.
 */
#ifndef KLC_MOE_H_
#define KLC_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KLC_ABI_VERSION 1

#define KLC_OK 0
#define KLC_ERR_ARGUMENT (-1)    /* null pointer or non-positive size */
#define KLC_ERR_SHAPE (-2)       /* a shape constraint is violated */
#define KLC_ERR_UNSUPPORTED (-3) /* valid but unsupported configuration */
#define KLC_ERR_HIP (-4)         /* HIP launch / runtime error */

#define KLC_DTYPE_BF16 0
#define KLC_DTYPE_F16 1
#define KLC_DTYPE_F32 2

#define KLC_PRECISION_FP32 0 /* expert_matmul_precision="fp32" */
#define KLC_PRECISION_BF16 1 /* expert_matmul_precision="bf16" */

/* Size limits of one call.  klc_moe_dispatch takes up to 2^21 (token, slot)
 * pairs (65535 tokens at k = 32); klc_moe_layer and the combines index tokens
 * by a grid dimension.  Longer inputs are split by the caller: tokens are
 * independent of each other along the whole path, so chunks give the same
 * bits as one call would. */
#define KLC_DISPATCH_MAX_PAIRS 2097152
#define KLC_LAYER_MAX_TOKENS 65535

/* Message for the last failing call on this thread ("" if none). */
const char* klc_last_error(void);
/* KLC_ABI_VERSION of the built library. */
int klc_abi_version(void);

/* ---- MXFP4 weights --------------------------------------------------------
 * Checkpoint layout (gpt-oss safetensors, read at mxfp4_expert.py:481-486):
 *   blocks[n_mat][out_dim][groups][16] uint8  (low nibble = even input column)
 *   scales[n_mat][out_dim][groups]     uint8  (E8M0, bias 127)
 */

/* Replaces dequantize_mxfp4_matrix (mxfp4_expert.py:357-379) for a batch of
 * n_mat matrices: writes out[n_mat][groups*32][out_dim] (the transposed
 * [in, out] layout) in out_dtype (KLC_DTYPE_*).  Bit-exact with torch.ldexp's
 * float32 product rounded to the dtype, including +-0, subnormals, +-inf and
 * the NaN of a zero code at scale 255. */
int klc_mxfp4_dequant(const void* blocks, const void* scales, void* out, int64_t n_mat, int64_t out_dim,
                      int64_t groups, int out_dtype, void* stream);

/* Bytes of one matrix in the packed row-tile layout consumed by the expert
 * kernels (out_dim must be a multiple of 64); negative on bad arguments. */
int64_t klc_mxfp4_packed_bytes(int64_t out_dim, int64_t groups);

/* Repacks checkpoint-layout matrices into the row-tile layout, matrix i at
 * packed + i * klc_mxfp4_packed_bytes(out_dim, groups).  Replaces the
 * host-side staging of _materialize_expert_matrix (mxfp4_expert.py:478-507),
 * which keeps the packed bytes instead of a dequantized copy. */
int klc_mxfp4_pack(const void* blocks, const void* scales, void* packed, int64_t n_mat, int64_t out_dim,
                   int64_t groups, void* stream);

/* dequantize_mxfp4_matrix (mxfp4_expert.py:357-379) applied to matrices held
 * in the packed layout (as Mxfp4ExpertStore.load_expert_matrix returns them,
 * mxfp4_expert.py:416-422); same output and semantics as klc_mxfp4_dequant. */
int klc_mxfp4_dequant_packed(const void* packed, void* out, int64_t n_mat, int64_t out_dim, int64_t groups,
                             int out_dtype, void* stream);

/* ---- Router -------------------------------------------------------------- */

/* Router logits, F.linear(hidden, W, b) in bfloat16
 * (streamed_moe_router.py:268-269): x[n_tokens][hidden], w[n_experts][hidden],
 * b[n_experts] bfloat16 -> logits[n_tokens][n_experts] bfloat16, computed as
 * bf16(f32(x . w) + b) with the dot product accumulated in float64.  If x_f32
 * is not NULL, also writes x as float32 [n_tokens][hidden] (hidden.float(),
 * streamed_moe_router.py:505). */
int klc_moe_router_logits(const void* x, const void* w, const void* b, void* logits, float* x_f32,
                          int64_t n_tokens, int64_t hidden, int64_t n_experts, void* stream);

/* Top-k selection and routing weights (streamed_moe_router.py:270-284,
 * 442-451, with routing locality disabled): per token, ids[t][j] (int32) of
 * the k largest logits in descending order (NaN largest), equal values in
 * the order torch.topk leaves them on the CPU (libstdc++ nth_element + sort,
 * or partial_sort when k * 64 <= n_experts), their float32 values, and
 * weights = torch's float32 CPU softmax over the k values rounded to
 * bfloat16.  k <= 32, n_experts <= 1024. */
int klc_moe_topk_softmax(const void* logits, int32_t* ids, float* values, void* weights, int64_t n_tokens,
                         int64_t n_experts, int64_t k, void* stream);

/* Routing weights for experts chosen on the host (streamed_moe_router.py:281-282
 * when routing locality is enabled and the selection of :331-394 is made by
 * the caller): weights[t][j] = bf16(softmax(values[t][:])[j]) as torch's
 * CPU softmax computes it in float32 (maximum propagating NaN, SLEEF expf,
 * sum in slot order, one reciprocal).  k <= 1024. */
int klc_moe_softmax_weights(const float* values, void* weights, int64_t n_tokens, int64_t k, void* stream);

/* Expert-sorted dispatch (no reference counterpart: the reference routes one
 * token per call, streamed_moe_router.py:499).  Pairs p = t*k + j are
 * counting-sorted by expert, ties by p: offsets[n_experts+1],
 * sorted_pairs[n_pairs], active[n_experts] (experts with >= 1 pair,
 * ascending, then -1 padding) and *n_active.  Also writes the work units of
 * the expert kernels, int32 units[klc_moe_units_size(n_pairs, n_experts)]:
 *   units[0..2] = number of decode gate_up (m = 8), decode down (m = 4) and
 *   prefill GEMM (m = 64) units, units[3] = 0, then the three lists in that
 *   order, with capacities C_m = (n_pairs + (m - 1) * min(n_pairs, n_experts)) / m.
 * A unit is expert | (pass << 10) and covers the pass-th run of m tokens of
 * that expert; experts ascending, then passes.
 * n_experts <= 256 and n_pairs <= KLC_DISPATCH_MAX_PAIRS.  Below 1024 pairs
 * one workgroup sorts; from 1024 on, one workgroup per expert counts every
 * expert and places its own expert's pairs, with the same outputs. */
int klc_moe_dispatch(const int32_t* ids, int64_t n_pairs, int64_t n_experts, int32_t* offsets,
                     int32_t* sorted_pairs, int32_t* active, int32_t* n_active, int32_t* units, void* stream);

/* Number of int32 elements of the dispatch's work-unit array (or a negative
 * status for unsupported sizes). */
int64_t klc_moe_units_size(int64_t n_pairs, int64_t n_experts);

/* ---- Experts ------------------------------------------------------------- */

/* gate_up GEMV + bias + clamped SwiGLU for every routed pair
 * (streamed_moe_router.py:500-506, 524-529).  w_gate_up is a device array of
 * n_experts pointers to packed [2*inter rows][hidden/32 groups] matrices;
 * bias is bfloat16 [n_experts][2*inter]; x is the bfloat16 hidden state
 * [n_tokens][hidden]; offsets, sorted_pairs and units are klc_moe_dispatch's
 * outputs for the n_tokens*k pairs.  Writes the down input to gated_split as
 * two bfloat16 planes [2][n_tokens*k][inter]: hi = bf16(y) and
 * lo = bf16(y - hi) of the float32 SwiGLU output y (under KLC_PRECISION_BF16,
 * where the reference rounds y to bfloat16, lo = 0), and, if gated_raw is not
 * NULL, y itself as float32 [n_tokens*k][inter].  hidden and inter must be
 * <= 3072, hidden a multiple of 64 and inter of 32. */
int klc_moe_gate_up(const void* const* w_gate_up, const void* bias, const void* x, int64_t n_tokens, int64_t k,
                    int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* units,
                    int64_t hidden, int64_t inter, float swiglu_limit, int precision, void* gated_split,
                    float* gated_raw, void* stream);

/* down GEMV + bias (streamed_moe_router.py:507-511): w_down is a device array
 * of n_experts pointers to packed [hidden rows][inter/32 groups] matrices;
 * bias bfloat16 [n_experts][hidden]; gated_split as written by
 * klc_moe_gate_up for n_pairs pairs -> expert_out[n_pairs][hidden] float32;
 * offsets, sorted_pairs and units from klc_moe_dispatch. */
int klc_moe_down(const void* const* w_down, const void* bias, const void* gated_split, int64_t n_pairs,
                 int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* units,
                 int64_t hidden, int64_t inter, int precision, float* expert_out, void* stream);

/* Weighted combine in top-k order (streamed_moe_router.py:497, 512-513):
 * out[t] = bf16 sum over j of bf16(bf16(expert_out[t*k+j]) * weights[t][j]),
 * every step rounded to bfloat16.  If residual (bfloat16 [n_tokens][hidden])
 * is not NULL, out[t] = bf16(residual[t] + out[t]), the residual add after the
 * MoE block (streamed_transformer_executor.py:260). */
int klc_moe_combine(const float* expert_out, const void* weights, const void* residual, int64_t n_tokens, int64_t k,
                    int64_t hidden, void* out, void* stream);

/* Bias-only fallback (streamed_moe_router.py:317-322):
 * out[t] = bf16(sum_j bf16(down_bias[ids[t][j]] * weights[t][j])), float32 sum. */
int klc_moe_bias_combine(const void* down_bias, const int32_t* ids, const void* weights, int64_t n_tokens,
                         int64_t k, int64_t hidden, void* out, void* stream);

/* L2 norms of the per-pair SwiGLU output and expert output, the expert_logs
 * diagnostics of streamed_moe_router.py:518-519: norms[p] = {|gated[p]|,
 * |expert_out[p]|}. */
int klc_moe_pair_norms(const float* gated, const float* expert_out, int64_t n_pairs, int64_t inter,
                       int64_t hidden, float* norms, void* stream);

/* ---- Prefill: expert-grouped GEMM ---------------------------------------------
 * The same expert math as klc_moe_gate_up / klc_moe_down (same arguments,
 * outputs and tolerance) for batches that give experts many tokens: the
 * dispatch's 64-token GEMM units x 256-row tiles, weights decoded in
 * registers into v_mfma_f32_16x16x32_bf16, activations staged in LDS. */
int klc_moe_gemm_gate_up(const void* const* w_gate_up, const void* bias, const void* x, int64_t n_tokens, int64_t k,
                         int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* units,
                         int64_t hidden, int64_t inter, float swiglu_limit, int precision, void* gated_split,
                         float* gated_raw, void* stream);

int klc_moe_gemm_down(const void* const* w_down, const void* bias, const void* gated_split, int64_t n_pairs,
                      int64_t n_experts, const int32_t* offsets, const int32_t* sorted_pairs, const int32_t* units,
                      int64_t hidden, int64_t inter, int precision, float* expert_out, void* stream);

/* ---- One MoE layer --------------------------------------------------------- */

/* Scratch bytes klc_moe_layer needs for n_tokens tokens.  The workspace must
 * be zero-filled once before its first use (it holds completion counters that
 * every call leaves at zero again); calls that share a workspace must be
 * ordered on one stream. */
int64_t klc_moe_workspace_bytes(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k);

/* One MoE layer for a batch of tokens — the route() + _execute_mxfp4_experts
 * path (streamed_moe_router.py:257-315, 483-522) for every row of x:
 * router logits -> top-k/softmax -> dispatch -> gate_up/SwiGLU -> down ->
 * combine, all enqueued on `stream` with no host synchronisation (batches of
 * up to 128 tokens run the router, top-k and dispatch as one launch).  Writes
 * out[n_tokens][hidden] bfloat16, plus residual (bfloat16 [n_tokens][hidden])
 * when that is not NULL (streamed_transformer_executor.py:260; out may alias
 * residual); ids/weights (optional, may be NULL) receive the routing.  workspace must be 256-byte aligned, hold
 * klc_moe_workspace_bytes() bytes and be zero-filled before its first use.  events: optional host array of
 * KLC_LAYER_EVENTS hipEvent_t handles recorded on `stream` before each of the
 * six kernels and after the last (NULL: no events); the one-launch path
 * records the first before its launch and the other six after it. */
#define KLC_LAYER_EVENTS 7
/* Expert path of klc_moe_layer.  AUTO picks the grouped GEMM once the batch
 * gives experts 8 or more tokens on average (n_tokens * k >= 8 * n_experts),
 * the decode GEMVs below that.  GEMV and GEMM force that expert path.  FUSED
 * runs the whole layer as one launch: batches of at most 16 tokens (at most
 * 64 token-slot pairs, 256 experts, k <= 16), 8-byte aligned out/residual,
 * and a stream that is not capturing a graph; other calls fail with
 * KLC_ERR_UNSUPPORTED.  It gives the same bits as GEMV.  Its workgroups wait
 * for one another (bounded spins on tagged flags), so it needs the compute
 * units to itself: do not run other work on the same GPU concurrently with a
 * FUSED launch (another stream, another process).  A wait that runs out
 * (KLC_FUSED_SPIN_LIMIT in the environment lowers the bound, for tests) sets
 * bit 0 of the workspace's status word (klc_moe_layer_status_offset) and
 * poisons that launch's outputs: ids -1, weights and out NaN. */
#define KLC_PATH_AUTO 0
#define KLC_PATH_GEMV 1
#define KLC_PATH_GEMM 2
#define KLC_PATH_FUSED 3
/* The path (KLC_PATH_GEMV, _GEMM or _FUSED) klc_moe_layer takes for these
 * sizes and `path` on `stream` with 8-byte aligned out/residual, or a
 * negative status.  No counterpart in the reference: it lets callers label
 * per-kernel timings (the one-launch layer records its events back to back). */
int klc_moe_layer_path(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, int path,
                       void* stream);
/* Byte offset, inside a klc_moe_layer workspace for these sizes, of the
 * one-launch layer's uint32 status word (-1 when the batch never runs as one
 * launch).  The word starts zero and keeps bit 0 set once a wait of some
 * launch ran out (which needs compute units held by other work for the whole
 * wait: the launch then completes with undefined outputs).  No counterpart
 * in the reference: a diagnostic for tests and monitoring. */
int64_t klc_moe_layer_status_offset(int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k);
int klc_moe_layer(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                  const void* gate_up_bias, const void* const* w_down, const void* down_bias, int64_t n_tokens,
                  int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, float swiglu_limit, int precision,
                  int path, void* workspace, int64_t workspace_bytes, void* out, const void* residual, int32_t* ids,
                  void* weights, void* const* events, void* stream);

/* route() of a layer whose experts are resident in HBM, with its expert_logs
 * (streamed_moe_router.py:257-329 calling _execute_mxfp4_experts, :483-522):
 * klc_moe_layer's work (no residual, no events; path AUTO, GEMV or GEMM —
 * FUSED fails with KLC_ERR_UNSUPPORTED) that also writes the routing to ids
 * (int32 [n_tokens][k]) and weights (bfloat16 [n_tokens][k]), the float32
 * SwiGLU outputs to gated ([n_tokens*k][inter]) and the expert_logs norms of
 * :518-519 to norms (float32 [n_tokens*k][2]: |gated|, |expert output|), all
 * from one call with no host synchronisation.  A caller that places ids,
 * weights and norms in one buffer reads the whole routing record back with
 * one copy.  Workspace as klc_moe_layer. */
int klc_moe_route(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                  const void* gate_up_bias, const void* const* w_down, const void* down_bias, int64_t n_tokens,
                  int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, float swiglu_limit, int precision,
                  int path, void* workspace, int64_t workspace_bytes, void* out, int32_t* ids, void* weights,
                  float* gated, float* norms, void* stream);

/* klc_moe_route with its routing record written to pinned host memory by
 * the GPU, for route() (streamed_moe_router.py:257-329), whose bookkeeping
 * (:296-329) needs only the selection: the kernel that selects the experts
 * also writes ids and weights into host_record, then `tag` into the record's
 * tag word; the norms kernel writes the norms there.  The host spins on the
 * tag word (cleared to 0 before the call) and books the selection while the
 * expert kernels still run, then synchronises `stream` for the norms.
 * host_record: pinned host memory mapped into the device (hipHostMalloc;
 * torch's pin_memory) of 4-byte words: ids (int32 [n_tokens*k]), weights
 * (bfloat16 [n_tokens*k], padded to a word), norms (float32 [n_tokens*k][2]),
 * the tag word.  tag: nonzero.  ids and weights are the device outputs as in
 * klc_moe_route; there is no device norms output. */
int klc_moe_route_readback(const void* x, const void* router_w, const void* router_b, const void* const* w_gate_up,
                           const void* gate_up_bias, const void* const* w_down, const void* down_bias,
                           int64_t n_tokens, int64_t hidden, int64_t inter, int64_t n_experts, int64_t k,
                           float swiglu_limit, int precision, int path, void* workspace, int64_t workspace_bytes,
                           void* out, int32_t* ids, void* weights, float* gated, void* host_record, uint32_t tag,
                           void* stream);

/* The selection half of route() (streamed_moe_router.py:268-284): router
 * logits -> top-k -> softmax weights for n_tokens rows, as klc_moe_layer
 * computes them (one launch for up to 128 tokens), into ids (int32
 * [n_tokens][k]) and weights (bfloat16 [n_tokens][k]).  For callers that need
 * the experts on the host before the expert kernels run (a streaming store
 * that must bring misses into HBM first).  workspace: a klc_moe_layer
 * workspace for these sizes (any intermediate size), zero-filled before its
 * first use. */
int klc_moe_select(const void* x, const void* router_w, const void* router_b, int64_t n_tokens, int64_t hidden,
                   int64_t n_experts, int64_t k, void* workspace, int64_t workspace_bytes, int32_t* ids,
                   void* weights, void* stream);

/* The expert half of route() for a selection made elsewhere
 * (_execute_mxfp4_experts, streamed_moe_router.py:483-522, once the experts
 * are known: the streaming store after it has brought misses into HBM, the
 * routing-locality path after its host-side selection): dispatch ->
 * gate_up/SwiGLU -> down -> combine (-> the expert_logs norms) for ids
 * (int32 [n_tokens][k], each in [0, n_experts)) and bfloat16 weights
 * [n_tokens][k], as klc_moe_layer runs them after its router.  gated and
 * norms are both NULL (no norms) or both set (as klc_moe_route).  path AUTO,
 * GEMV or GEMM; workspace as klc_moe_layer. */
int klc_moe_experts(const void* x, const int32_t* ids, const void* weights, const void* const* w_gate_up,
                    const void* gate_up_bias, const void* const* w_down, const void* down_bias, int64_t n_tokens,
                    int64_t hidden, int64_t inter, int64_t n_experts, int64_t k, float swiglu_limit, int precision,
                    int path, void* workspace, int64_t workspace_bytes, void* out, float* gated, float* norms,
                    void* stream);

/* The same layer as klc_moe_layer without a workspace argument: it has no
 * counterpart in the reference and is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc).  It calls no hipMalloc, hipFree or allocating routine.
 * Its scratch is a static device array of KLC_STATIC_SCRATCH_BYTES in the
 * library, one per GPU, held until the process ends; a call needing more
 * (klc_moe_workspace_bytes(n_tokens, ...) > KLC_STATIC_SCRATCH_BYTES: at
 * gpt-oss-120B shape, more than about 360 tokens) fails with
 * KLC_ERR_UNSUPPORTED.  Every call on one GPU shares that GPU's array, so
 * calls that overlap on one GPU (different streams, or threads without
 * ordering) race: order them on one stream.  The first call on a device
 * looks the array up and clears its counters with a kernel on `stream`.
 * Arguments and results as klc_moe_layer. */
#define KLC_STATIC_SCRATCH_BYTES (32 * 1024 * 1024)
int klc_moe_layer_static_scratch(const void* x, const void* router_w, const void* router_b,
                                 const void* const* w_gate_up, const void* gate_up_bias, const void* const* w_down,
                                 const void* down_bias, int64_t n_tokens, int64_t hidden, int64_t inter,
                                 int64_t n_experts, int64_t k, float swiglu_limit, int precision, int path, void* out,
                                 const void* residual, int32_t* ids, void* weights, void* const* events, void* stream);

/* ---- RMSNorm (stacked decode) -------------------------------------------------
 * rms_norm(x, weight, eps) of streamed_attention.py:27-28 for bfloat16
 * x[n_tokens][hidden] and weight[hidden]: x * rsqrt(mean(x.float()^2) + eps)
 * .to(bfloat16) * weight, with the mean of squares rounded to float32 and each
 * multiply rounded to bfloat16.  hidden a multiple of 8, <= 8192. */
int klc_rms_norm(const void* x, const void* weight, void* out, int64_t n_tokens, int64_t hidden, float eps,
                 void* stream);

/* ---- Safetensors shards (expert store misses) ----------------------------------
 * Replace the per-miss safe_open(...).get_slice(name)[expert] -> pin_memory()
 * -> .to(device) chain of Mxfp4ExpertStore._load_expert_tensor /
 * _materialize_expert_matrix (mxfp4_expert.py:478-525) and the shard lookups of
 * SafetensorIndex (streamed_loader.py:43-82).  A shard is opened and its
 * header parsed once (klc_st_open; *handle is an opaque pointer, released by
 * klc_st_close; lookups are read-only, so threads may share a handle).
 * Rows [first, first + count) along dimension 0 of a tensor -- one expert of
 * a [E, ...] tensor -- are one contiguous byte range.
 * klc_st_tensor_info: dtype string (<= 15 chars, e.g. "U8", "BF16"), shape
 * (up to 8 dims), absolute byte offset in the file and byte size.  Missing
 * names give KLC_ERR_ARGUMENT; malformed headers KLC_ERR_SHAPE. */
int klc_st_open(const char* path, void** handle);
int klc_st_close(void* handle);
int klc_st_tensor_info(void* handle, const char* name, char* dtype, int64_t* shape, int* ndim, int64_t* data_offset,
                       int64_t* nbytes);
/* rows [first, first + count) into host memory, read with pread by a pool of
 * up to 8 threads */
int klc_st_read_rows(void* handle, const char* name, int64_t first, int64_t count, void* dst);
/* the same rows into device memory: read into a ring of pinned staging slots
 * (at most 2 MiB each; staging_bytes >= 8 KiB) and copied with hipMemcpyAsync
 * on `stream`; a slot is refilled once its previous copy has read it, so
 * reads overlap PCIe copies.  Returns once the staging buffer is free again
 * (every device copy is then complete). */
int klc_st_copy_rows_to_device(void* handle, const char* name, int64_t first, int64_t count, void* staging,
                               int64_t staging_bytes, void* dst, void* stream);
/* n row ranges (names[i], firsts[i], counts[i]) -> dsts[i] through one ring
 * and one final wait: an expert's blocks and scales in a single call */
int klc_st_copy_rows_batch(void* handle, int n, const char* const* names, const int64_t* firsts,
                           const int64_t* counts, void* const* dsts, void* staging, int64_t staging_bytes,
                           void* stream);
/* One expert's MXFP4 projection from the shard straight into the packed
 * row-tile layout in device memory (what klc_mxfp4_pack makes): blocks
 * [E, rows, G, 16] and scales [E, rows, G], both U8 in this shard, expert
 * `expert`, rows a multiple of 64.  Chunks of whole 64-row tiles are read
 * (pread by the pool) into the slots of a ring in the pinned host staging
 * buffer, and a pack kernel on `stream` reads each slot over PCIe and writes
 * its tiles of `packed`.  Asynchronous: returns once every chunk is read and
 * its pack enqueued; `packed` is complete when `stream` reaches the last
 * pack.  The staging buffer stays in use until then: a later call with the
 * same buffer waits for a slot's pack before refilling it (so consecutive
 * loads overlap), klc_st_copy_rows_* wait for all of them, and
 * klc_st_staging_wait / klc_st_staging_release must be called before the
 * buffer is freed or used otherwise.  One thread fills a buffer at a time.
 * staging: pinned host memory (hipHostMalloc / torch pin_memory) of
 * staging_bytes, at least two tiles (2 * 64 * G * 17 bytes); staging and
 * packed 16-byte aligned; packed holds klc_mxfp4_packed_bytes(rows, G). */
int klc_st_load_mxfp4_packed(void* handle, const char* blocks_name, const char* scales_name, int64_t expert,
                             void* staging, int64_t staging_bytes, void* packed, void* stream);
/* Waits (host) for every pack still reading the staging buffer. */
int klc_st_staging_wait(const void* staging);
/* klc_st_staging_wait, then forgets the buffer's ring (its events are
 * destroyed); call before freeing a staging buffer. */
int klc_st_staging_release(const void* staging);

/* ---- lm_head ---------------------------------------------------------------
 * Replaces StreamedTransformerExecutor.logits (streamed_transformer_executor.py:177-209:
 * float32 matmul of 4096-row chunks of the resident lm_head weight with the
 * final hidden state, each chunk copied to the host) and the greedy pick of
 * its callers (generation_runtime.py:118-122, inference_server.py:383-386:
 * nan_to_num(nan=-1e9, posinf=1e9, neginf=-1e9), then argmax).
 * w: bfloat16 [vocab][hidden]; x: float32 [hidden] (hidden.float()).
 * logits[v] = f32(sum_h f64(w[v][h]) * f64(x[h])), the correctly rounded
 * float32 dot product; *token = the first index of the largest
 * nan_to_num(logits[v]), *token_logit (may be NULL) that value.
 * hidden a multiple of 8, at most 4096; w, x, workspace 16-byte aligned;
 * workspace of klc_lm_head_workspace_bytes(vocab) bytes (scratch, no
 * initialisation needed). */
int64_t klc_lm_head_workspace_bytes(int64_t vocab);
int klc_lm_head_logits(const void* w, const float* x, float* logits, int64_t vocab, int64_t hidden, void* workspace,
                       int64_t workspace_bytes, int32_t* token, float* token_logit, void* stream);

/* ---- Decode attention ------------------------------------------------------
 * One decode token of StreamedAttention.forward (streamed_attention.py:80-141)
 * on a device-resident KV ring (kv_cache_manager.py:39-56 keeps a list and
 * stacks it every step).  The ring of a layer holds k_cache and v_cache,
 * [cap][n_kv][head_dim] of kv_dtype (KLC_DTYPE_F16, the reference's "fp16"
 * default, or KLC_DTYPE_BF16); token n lives in slot n % cap.  q, k, v and
 * the context are bfloat16. */
/* apply_rope (:88-98) to q [n_heads][head_dim] -> q_out (may alias q) and to
 * k [n_kv][head_dim] -> k_cache slot `slot` (and, if k_out is not NULL, the
 * rotated bfloat16 key to k_out); v is stored to v_cache slot `slot`.  cos_half / sin_half: bfloat16 [head_dim / 2] of the position
 * (rope_cos_sin, :81-85).  Every bfloat16 op rounds as torch's does. */
int klc_rope_append(const void* q, const void* k, const void* v, const void* cos_half, const void* sin_half,
                    void* q_out, void* k_out, void* k_cache, void* v_cache, int64_t slot, int64_t cap, int64_t n_heads,
                    int64_t n_kv, int64_t head_dim, int kv_dtype, void* stream);
/* Scratch bytes of klc_attn_decode for `count` keys. */
int64_t klc_attn_workspace_bytes(int64_t n_heads, int64_t head_dim, int64_t count);
/* context [n_heads][head_dim] bfloat16 from the `count` keys starting at ring
 * slot `first` (in token order, wrapping at cap) -- the caller applies the
 * sliding window by choosing them.  scores = f32(q . k) / sqrt(head_dim);
 * softmax over [scores, sinks[h]] (sinks bfloat16 [n_heads], or NULL) with
 * the maximum subtracted; probabilities rounded to kv_dtype; context =
 * bf16(kv_dtype(sum p * v)).  head_dim a multiple of 8 up to 128; n_heads / n_kv <= 16;
 * count <= 2^22; caches and workspace 16-byte aligned. */
int klc_attn_decode(const void* q, const void* k_cache, const void* v_cache, const void* sinks, int64_t cap,
                    int64_t first, int64_t count, int64_t n_heads, int64_t n_kv, int64_t head_dim, int kv_dtype,
                    void* workspace, int64_t workspace_bytes, void* context, void* stream);

/* ---- Synthetic inputs -------------------------------------------------------
 * Counter-based SplitMix64 stream, identical to klcquant_amd/synth.py:
 * mode 0: n random bytes; mode 1: n bytes uniform in [lo, hi]. */
int klc_synth_fill(void* dst, int64_t n, uint64_t seed, int mode, int lo, int hi, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KLC_MOE_H_ */
