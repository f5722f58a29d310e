/*
 * cx_moe.h — C ABI of the MI355X (gfx950) MoE expert-compute engine.
 *
 * This is the drop-in boundary for Constellation's routed-expert hot path.
 * Every entry point takes plain pointers and sizes, returns an int status
 * (CX_OK == 0, negative on error; cx_last_error() gives the message for the
 * calling thread) and never throws.  Device pointers are raw HIP device
 * addresses; `stream` is a hipStream_t passed as void* (NULL = the legacy
 * default stream).
 *
 * Threading: the per-device upload arena is process-wide and locked, so
 * cx_upload_matrix / cx_free_device may run on a different thread than the
 * compute calls (the reference uploads on its `resident_bg` thread while the
 * worker thread serves inference, expert_node_v2/control.cc:130-276 and
 * expert_node_v2/worker.cc:142-275).  A cx_ctx holds per-worker scratch and
 * is used by one thread at a time; every call makes its device current
 * itself (the reference does the same at backend_cuda_v2.cc:102 and
 * backend_workspace_cuda_v2.cc:149).
 */
#ifndef CX_MOE_H_
#define CX_MOE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#define CX_API __attribute__((visibility("default")))
#else
#define CX_API
#endif

/* ---- status codes -------------------------------------------------------- */
enum {
    CX_OK = 0,
    CX_EINVAL = -1,       /* bad argument / shape / dtype                     */
    CX_ENOMEM = -2,       /* HBM arena or pinned staging exhausted            */
    CX_EHIP = -3,         /* a HIP runtime call failed                        */
    CX_EUNSUPPORTED = -4, /* valid request the engine does not implement      */
    CX_EDEVICE = -5       /* device-side check failed (bad expert id, ...)    */
};

/* Activation dtypes.  1 and 2 are the wire values of common::ActivationDType
 * (common/protocol.h:48-52); 3 is fp32, used by the router and parity outputs. */
enum { CX_DTYPE_FP16 = 1, CX_DTYPE_BF16 = 2, CX_DTYPE_F32 = 3 };

CX_API const char* cx_last_error(void);
CX_API const char* cx_version(void);

/* ---- device probes --------------------------------------------------------
 * Replace BuildLocalAmdGpuInfosV2 / BuildLocalAmdDynamicGpuInfosV2, the stubs
 * at expert_node_v2/backend/amd/gpu_info_amd_v2.cc:3-21 (contract:
 * backend_registry_v2.h:12-19).  The glue maps these fields onto
 * common::StaticGpuInfo / DynamicGpuInfo (common/types.h:85-110). */
typedef struct cx_device_info {
    char name[128];          /* marketing name, e.g. "AMD Instinct MI355X"; "AMD gfx950" when the host has no name table */
    char arch[64];           /* gcnArchName, e.g. "gfx950:sramecc+:xnack-"  */
    uint64_t total_mem_bytes;
    uint64_t free_mem_bytes;
    uint32_t capability_flags; /* kGpuCapFp16|kGpuCapBf16|kGpuCapFp8 (types.h:76-78) */
    int32_t compute_units;
    int32_t num_xcds;          /* best effort; 0 when the runtime does not say */
} cx_device_info;

CX_API int cx_device_count(int* count);
CX_API int cx_device_query(int device, cx_device_info* out);

/* ---- expert residency ----------------------------------------------------
 * One fp8-e4m3fn matrix with fp32 block scales (`scale_inv`, multiply to
 * dequantize), row-major [rows, cols], scales row-major
 * [ceil(rows/row_block), ceil(cols/col_block)] — the layout validated by
 * BuildMatrixBlockScaleViewV2 (expert_node_v2/expert_format_v2.cc:68-139).
 *
 * cx_upload_matrix replaces the per-tensor cudaMalloc+cudaMemcpy of
 * UploadSpanToCuda (backend/cuda/backend_cuda_v2.cc:14-53) with a
 * sub-allocation from a per-device HBM arena, then canonicalises the two
 * non-finite OCP codes 0x7F/0xFF to 0x7E/0xFE: the reference decoder maps
 * both to +-448 (backend/fp8_lut_v2.cc:61), which 0x7E/0xFE also encode, so
 * the hardware OCP converter then reproduces the reference values exactly.
 * Any shape and block size is accepted (the reference's control tests send
 * 4x8 matrices with 1x1 blocks); only the kernels specialise.
 * Host pointers in, device pointers out.  Synchronous. */
CX_API int cx_upload_matrix(int device,
                     const uint8_t* host_weight, uint64_t rows, uint64_t cols,
                     const float* host_scale, uint64_t scale_count,
                     uint8_t** dev_weight, float** dev_scale);

/* The same upload with the weight re-tiled on the device for the gate/up
 * kernels (CX_LAYOUT_TILE16: 2 KB tiles of 16 rows x 128 columns, the tiles
 * of a 16-row group in column order; inside a tile the 32 bytes of row r,
 * columns 32q..32q+31 at (16q + r) * 32), so that each wave's weight range
 * is contiguous in HBM.  The wire bytes, the scales and the result of every
 * kernel are unchanged; rows % 16 == 0 and cols % 128 == 0 are required.
 * Mark the descriptor's gu_layout CX_LAYOUT_TILE16 for an expert whose up
 * and gate came this way.  No counterpart in the reference: its CUDA
 * upload (backend/cuda/backend_cuda_v2.cc:94-145) keeps all three matrices
 * row-major; this library's UploadExpertAmdV2 calls this entry for w_up and
 * w_gate when the shape allows. */
CX_API int cx_upload_matrix_tiled(int device,
                     const uint8_t* host_weight, uint64_t rows, uint64_t cols,
                     const float* host_scale, uint64_t scale_count,
                     uint8_t** dev_weight, float** dev_scale);

/* Release one arena sub-allocation made by this library (weight or scale).
 * device < 0 searches every device's arena for the pointer (the reference's
 * FreeDeviceBuffer takes no device either).  NULL is a no-op.  Like
 * cudaFree, it first waits for all work queued on the device, so kernels
 * still reading the range (another thread's inference) finish before a later
 * upload can reuse it; the calling thread's current device is left as it was.
 * Replaces FreeDeviceBuffer (backend/cuda/backend_cuda_v2.cc:55-65). */
CX_API int cx_free_device(int device, void* dev_ptr);

/* Bytes currently sub-allocated / reserved by the device's arena. */
CX_API int cx_arena_stats(int device, uint64_t* used_bytes, uint64_t* reserved_bytes);

/* Device-resident expert, the plain-pointer image of ExpertDeviceStorageV2
 * (expert_node_v2/expert_format_v2.h:170-237):
 *   up, gate: [inter, hidden];  down: [hidden, inter]  (HF nn.Linear [out,in]).
 * *_rb / *_cb are the row/col block sizes of each matrix's scale grid.
 * gu_layout: how w_up and w_gate sit in HBM, CX_LAYOUT_ROWS (row-major, the
 * wire order) or CX_LAYOUT_TILE16 (cx_upload_matrix_tiled; the scales stay
 * row-major).  w_down is always row-major. */
#define CX_LAYOUT_ROWS 0
#define CX_LAYOUT_TILE16 1
typedef struct cx_expert_desc {
    const uint8_t* w_up;   const float* s_up;
    const uint8_t* w_gate; const float* s_gate;
    const uint8_t* w_down; const float* s_down;
    int32_t hidden;        /* 7168 for DeepSeek-V3 */
    int32_t inter;         /* 2048 */
    int32_t up_rb, up_cb, gate_rb, gate_cb, down_rb, down_cb;
    int32_t gu_layout;     /* CX_LAYOUT_ROWS or CX_LAYOUT_TILE16 */
    int32_t reserved[3];   /* zero */
} cx_expert_desc;

/* ---- per-worker context -------------------------------------------------- */
typedef struct cx_ctx cx_ctx;
CX_API int cx_ctx_create(int device, cx_ctx** out);
CX_API int cx_ctx_destroy(cx_ctx* ctx);
/* Waits for the context's work on `stream` and reports any device-side
 * check that failed since the last call (CX_EDEVICE, message in
 * cx_last_error). */
CX_API int cx_ctx_sync(cx_ctx* ctx, void* stream);

/* Per-kernel timing with HIP events recorded on the launch stream around
 * every kernel the context launches (kernels: "route", "plan", "gate_up",
 * "down", "combine").  cx_ctx_profile(ctx, 1) starts collecting (and clears
 * totals), 0 stops.  cx_ctx_profile_read synchronises on the recorded events
 * and returns the launch count and summed milliseconds of one kernel. */
CX_API int cx_ctx_profile(cx_ctx* ctx, int enable);
CX_API int cx_ctx_profile_read(cx_ctx* ctx, const char* kernel, int* launches,
                        double* total_ms);

/* ---- one expert, B tokens (device pointers) -------------------------------
 * y = down( silu(gate.x) * (up.x) ), fp32 accumulation, h kept in fp32,
 * output cast to out_dtype with round-to-nearest-even; y_f32 (nullable)
 * receives the fp32 pre-cast output for parity checks.
 * Semantics of RunExpertCudaV2 (backend/cuda/backend_cuda_v2.cc:205-255)
 * and RunExpertReferenceV2 (backend/expert_reference_v2.cc:146-178), with
 * batch >= 1 instead of the reference's batch == 1
 * (backend_workspace_cuda_v2.cc:146) and both fp16 and bf16 in/out. */
CX_API int cx_expert_run(cx_ctx* ctx, const cx_expert_desc* expert,
                  const void* x, int in_dtype, int n_tokens,
                  void* y, int out_dtype, float* y_f32, void* stream);

/* Allocation-free variant of cx_expert_run.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory — code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.  It takes no
 * context and never calls hipMalloc, hipFree or an allocating library
 * routine; its scratch (h, or the k-part gate/up sums at 1..4 tokens) is a
 * static device array of CX_STATIC_SCRATCH_BYTES that each GPU holds until the
 * process ends.  Same kernels and results as cx_expert_run.
 * Limit: the path's scratch must fit in CX_STATIC_SCRATCH_BYTES — 16 bytes
 * per (token, inter row) at 1..4 tokens, 4 bytes (plus up to 256 of
 * alignment) otherwise; at DeepSeek-V3's inter 2048 that is up to 32 tokens.
 * A larger call returns CX_EINVAL.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (two streams, two threads) race;
 * serialise them.  Nothing in the array has to start at zero: each call
 * writes what it reads. */
#define CX_STATIC_SCRATCH_BYTES (256 * 1024)
CX_API int cx_expert_run_static(int device, const cx_expert_desc* expert,
                         const void* x, int in_dtype, int n_tokens,
                         void* y, int out_dtype, float* y_f32, void* stream);

/* Host-buffer variant with the exact contract of
 * BackendWorkspaceV2::RunExpertRequest (backend/backend_workspace_v2.h:18-21)
 * as implemented for CUDA at backend_workspace_cuda_v2.cc:26-109/139-182:
 * x_bytes must equal n_tokens*hidden*sizeof(in_dtype), y receives
 * n_tokens*hidden*sizeof(out_dtype) bytes.  Uses persistent device and
 * pinned staging buffers of the context (no per-request hipMalloc) and
 * returns after the output is on the host. */
CX_API int cx_expert_run_host(cx_ctx* ctx, const cx_expert_desc* expert,
                       const void* x_host, size_t x_bytes, int in_dtype,
                       int n_tokens, void* y_host, size_t y_bytes,
                       int out_dtype);

/* ---- MoE layer ------------------------------------------------------------
 * A layer is a device table of up to n_experts resident experts indexed by
 * local expert id (0..n_experts-1; NULL entries = not resident) plus an
 * optional shared expert applied to every token with weight 1.0.
 * The routed ids are local expert ids, as produced by route_token_real
 * (server/moe_layer_runtime.py:366-384) before make_global_expert_id. */
typedef struct cx_layer cx_layer;
CX_API int cx_layer_create(cx_ctx* ctx, int n_experts,
                    const cx_expert_desc* const* experts,
                    const cx_expert_desc* shared, cx_layer** out);
CX_API int cx_layer_destroy(cx_ctx* ctx, cx_layer* layer);

/* DeepSeek-V3 router (noaux_tc, sigmoid), server/moe_layer_runtime.py:232-408:
 *   logits = W_r . x ; s = sigmoid(logits) ; c = s + bias (masked -> -inf)
 *   group score = sum of top-2 of c per group; keep topk_group groups;
 *   top_k of c inside kept groups (k = min(top_k, #resident));
 *   w = s[idx]; if norm && k>1: w /= (sum w + 1e-20); w *= scale.
 * x: [n_tokens, hidden] (bf16 or fp32), w_router: [n_experts, hidden]
 * (bf16 or fp32), bias: fp32 [n_experts], resident: uint8 [n_experts] or
 * NULL (all resident).  Logits accumulate exact products in fp64 and the
 * selection runs in fp64, so the chosen sets equal the exact-math result.
 * Ties break toward the lower expert index.  Outputs, per token, in
 * descending choice-score order: topk_ids int32 [n_tokens, top_k] and
 * topk_w fp32 [n_tokens, top_k]; slots beyond min(top_k, #resident) get
 * id -1, weight 0. */
CX_API int cx_route(cx_ctx* ctx, const void* x, int x_dtype,
             const void* w_router, int w_dtype, const float* bias,
             const uint8_t* resident, int n_tokens, int hidden, int n_experts,
             int n_group, int topk_group, int top_k, int norm_topk_prob,
             float routed_scaling_factor, int32_t* topk_ids, float* topk_w,
             void* stream);

/* Copies the fp64 router logits W_r . x [n_tokens, n_experts] of the
 * context's most recent router call (cx_route or cx_moe_layer) into `out`
 * (device memory), ordered on `stream` after that call.  For the diagnostic
 * fields route_token_real returns with return_aux=True (logits, scores,
 * group scores; server/moe_layer_runtime.py:386-407).  CX_EINVAL when the
 * shape differs from the last call's. */
CX_API int cx_route_logits(cx_ctx* ctx, double* out, int n_tokens, int n_experts,
                    void* stream);

/* Routed-expert compute for a token batch: every active expert and the
 * shared expert of the layer in grouped launches, with per-expert token
 * gather and a deterministic weighted combine (fp32, route order, shared
 * last) — a3+a4+a5+a9..a12 of the reference's decode path
 * (moe_layer_runtime.py:111-167, deepseek_full_model_executor.py:264-316,
 * full_model_runtime.py:348).  Negative ids are skipped; an id that is out
 * of range or not resident, an expert listed twice for one token, and a
 * negative or non-finite route weight (the checks of validate_routes,
 * server/moe_layer_runtime.py:84-98) set the context's device error
 * (reported by cx_ctx_sync) and the route is skipped.  The checks run in the
 * planner on the device, so no route ever travels to the host.
 * cx_moe_decode targets n_tokens <= 16 per launch set;
 * cx_moe_prefill targets larger chunks (grouped MFMA GEMM tiles of 16
 * tokens, up to 64 tokens per work item).  Both accept any n_tokens. */
CX_API int cx_moe_decode(cx_ctx* ctx, const cx_layer* layer,
                  const void* x, int in_dtype, int n_tokens,
                  const int32_t* topk_ids, const float* topk_w, int top_k,
                  void* y, int out_dtype, float* y_f32, void* stream);
CX_API int cx_moe_prefill(cx_ctx* ctx, const cx_layer* layer,
                   const void* x, int in_dtype, int n_tokens,
                   const int32_t* topk_ids, const float* topk_w, int top_k,
                   void* y, int out_dtype, float* y_f32, void* stream);

/* Router + routed experts + shared expert in one call (device pointers);
 * topk_ids / topk_w (nullable) receive the routing decision. */
CX_API int cx_moe_layer(cx_ctx* ctx, const cx_layer* layer,
                 const void* x, int in_dtype, int n_tokens,
                 const void* w_router, int w_dtype, const float* bias,
                 const uint8_t* resident, int n_group, int topk_group,
                 int top_k, int norm_topk_prob, float routed_scaling_factor,
                 void* y, int out_dtype, float* y_f32,
                 int32_t* topk_ids, float* topk_w, void* stream);

/* ---- whole-layer wire message ---------------------------------------------
 * MoeLayerRequest (msg_type 42) / MoeLayerResponse (43): one request per
 * node per layer instead of one InferRequest per selected expert, sent
 * sequentially (moe_layer_runtime.py:111-145, infer_one_expert :27-81).  No
 * counterpart in the reference's v1 protocol (common/protocol.h:13-37); the
 * types are additive and v1 InferRequest/InferResponse stay byte-identical.
 * Little-endian bodies in the style of common/infer_codec.cc:7-76:
 *   request:  i32 layer_id, i32 batch_size T, i32 hidden_dim H, i32 top_k K,
 *             u32 input_dtype, u32 output_dtype (ActivationDType: 1 fp16,
 *             2 bf16), u32 flags (bit 0: add the layer's shared expert),
 *             u32 n_routes (= T*K), i32 expert_ids[n_routes] (local ids of the
 *             layer, -1 = no expert on this node), f32 expert_weights[n_routes],
 *             u32 activation_nbytes (= T*H*2), activation bytes [T, H].
 *   response: i32 status_code (0 ok, 1 expert unknown, 2 expert not resident,
 *             4 execution failure: the codes of worker.cc:113-132),
 *             i32 batch_size, i32 hidden_dim, u32 output_dtype,
 *             u32 output_nbytes (T*H*2, or 0 on failure), output bytes [T, H]:
 *             y[t] = sum_k w[t][k] * expert_k(x[t]) in route order, then
 *             + shared(x[t]) (combine_outputs_torch, moe_layer_runtime.py:
 *             148-167, and full_model_runtime.py:348), in fp32, rounded once. */
#define CX_MSG_MOE_LAYER_REQUEST 42
#define CX_MSG_MOE_LAYER_RESPONSE 43
#define CX_MOE_LAYER_FLAG_SHARED 1u

typedef struct cx_moe_layer_request_info {
    int32_t layer_id, batch_size, hidden_dim, top_k;
    uint32_t input_dtype, output_dtype, flags;
} cx_moe_layer_request_info;

/* Validates a request body (exact length, field ranges) and returns its
 * header fields, so a worker can pick the layer before running it.  Host
 * only. */
CX_API int cx_moe_layer_request_peek(const uint8_t* body, size_t body_len,
                              cx_moe_layer_request_info* out);
/* Bytes of a full (status 0) response body for T tokens of hidden H. */
CX_API size_t cx_moe_layer_response_size(int batch_size, int hidden_dim);
/* Runs one request body against `layer` (whose entry i is the layer's local
 * expert i on this node) through persistent pinned and device buffers: one
 * host->device copy of routes + activation, cx_moe_decode (T <= 16) or
 * cx_moe_prefill, one device->host copy.  Writes the response body into
 * resp[resp_cap] (resp_cap >= cx_moe_layer_response_size) and its length
 * into *resp_len.  Request-level failures (unknown / non-resident expert,
 * hidden mismatch, a negative or non-finite route weight — rejected like
 * validate_routes, server/moe_layer_runtime.py:96-97 — or a device check)
 * become a status code in the response
 * and CX_OK; a malformed body or an undersized buffer returns CX_EINVAL
 * without a response. */
CX_API int cx_moe_layer_request_run(cx_ctx* ctx, const cx_layer* layer,
                             const uint8_t* body, size_t body_len,
                             uint8_t* resp, size_t resp_cap, size_t* resp_len);

/* ---- synthetic data ------------------------------------------------------
 * Counter-based generator shared bit-for-bit with the CPU oracle, so any
 * single tensor can be regenerated on either side:
 *   v[i] = std * N(seed, stream, i)     (Box-Muller on a splitmix64 hash)
 * cx_gen_fp8_matrix quantises per row_block x col_block block:
 *   scale = max(amax/448, 1e-12), q = e4m3fn_rne_saturate(v/scale).
 * Plays the role of FillDummyExpertBundleV2
 * (backend/dummy_expert_data_v2.cc:9-132) for the benchmark shapes. */
CX_API int cx_gen_fp8_matrix(cx_ctx* ctx, uint64_t seed, uint64_t stream_id,
                      int rows, int cols, int row_block, int col_block,
                      float std_dev, uint8_t* dev_weight, float* dev_scale,
                      void* stream);
/* dtype CX_DTYPE_BF16 / FP16 (RNE from fp32) or CX_DTYPE_F32. */
CX_API int cx_gen_normal(cx_ctx* ctx, uint64_t seed, uint64_t stream_id,
                  uint64_t count, float std_dev, int dtype, void* dev_out,
                  void* stream);
/* Allocate (arena) and generate a whole expert (hidden x inter, blocks).
 * Up and gate are written in CX_LAYOUT_TILE16 when inter % 16 == 0 and
 * hidden % 128 == 0 (out->gu_layout says which); the values are the same. */
CX_API int cx_gen_expert(int device, uint64_t seed, uint64_t stream_base,
                  int hidden, int inter, int block, float std_dev,
                  cx_expert_desc* out);
/* Free the six arena buffers of an expert made by cx_gen_expert or by
 * cx_upload_matrix / cx_upload_matrix_tiled calls, and zero the descriptor. */
CX_API int cx_free_expert(int device, cx_expert_desc* expert);

#ifdef __cplusplus
}
#endif
#endif /* CX_MOE_H_ */
