/*
 * l0hip: MI355X (gfx950) implementation of the l0llm decoder matmul and
 * decode-attention path, behind a plain C ABI.
 *
 * The reference (hf-laboratories/l0llm) is C#; its kernels come from the
 * external LevelZero.NET package, consumed through LevelZero.ComputeDevice,
 * SharedBuffer<T>, LevelZeroRuntime and LevelZero.Kernels.LlmKernelSuite.
 * Each entry point below names the reference member it replaces, with the
 * call site (file:line, relative to src/HFLabs.ML.LLM.LevelZero/ unless a
 * path is given) that fixes its argument order and meaning. A C# P/Invoke
 * shim maps these onto the LevelZero-shaped classes.
 *
 * Conventions
 *  - Every function returns an int status: L0H_OK (0) or a negative L0H_ERR_*
 *    code; l0h_last_error() returns the calling thread's message for the last
 *    failure. The codes map onto the .NET exceptions the reference throws.
 *  - Pointers named x, y, q, k, v, w, table, logits, ... are DEVICE pointers
 *    obtained from l0h_alloc (or from a matrix/model object). Host pointers
 *    are named host_*.
 *  - All sizes are element counts (int, as the reference) unless named *_bytes.
 *  - Outside recording, operations are enqueued in order on the device's
 *    stream; l0h_read and l0h_synchronize wait for them. Between
 *    l0h_begin_recording and l0h_end_recording they are captured into one HIP
 *    graph, launched and waited for at l0h_end_recording.
 *  - Calls may come from any thread; every entry point selects its device.
 */
#ifndef L0HIP_H
#define L0HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ----------------------------------------------------- */
#define L0H_OK 0
#define L0H_ERR_INVALID_ARG (-1)    /* ArgumentException / ArgumentNull / ArgumentOutOfRange */
#define L0H_ERR_UNSUPPORTED (-2)    /* NotSupportedException */
#define L0H_ERR_INVALID_OP (-3)     /* InvalidOperationException */
#define L0H_ERR_INVALID_DATA (-4)   /* InvalidDataException */
#define L0H_ERR_OUT_OF_MEMORY (-5)  /* allocation failure */
#define L0H_ERR_DEVICE (-6)         /* HIP runtime / device failure */

/* ---- element types ---------------------------------------------------- */
#define L0H_F32 0
#define L0H_F16 1
#define L0H_BF16 2
#define L0H_I8PC 3 /* int8 weight-only, one fp16 scale per output row */

/* ---- LlmWeightPrecision (LlmWeightPrecision.cs:3-19), plus BFloat16 ---- */
#define L0H_PRECISION_AUTO 0
#define L0H_PRECISION_FLOAT32 1
#define L0H_PRECISION_FLOAT16 2
#define L0H_PRECISION_INT8 3
#define L0H_PRECISION_BFLOAT16 4

typedef struct l0h_device l0h_device;
typedef struct l0h_matrix l0h_matrix;
typedef struct l0h_model l0h_model;

/* ======================================================================
 * Device runtime (replaces LevelZero.LevelZeroRuntime / ComputeDevice /
 * SharedBuffer<T>)
 * ==================================================================== */

/* LevelZeroRuntime.IsAvailable (LevelZeroLlmEngine.cs:355-360): 1 if a gfx950 device is present. */
int l0h_runtime_is_available(void);
/* LevelZeroRuntime.EnumerateDevices (../l0llm/Program.cs:124): number of HIP devices. */
int l0h_device_count(int* count);
/* LevelZeroRuntime.GetDevice(0, id) (LevelZeroLlmEngine.cs:359). */
int l0h_device_open(int ordinal, l0h_device** out);
/* ComputeDevice.Dispose. */
int l0h_device_close(l0h_device* dev);
/* Device name and compute-unit count (../l0llm/Program.cs:138 prints the device). */
int l0h_device_info(l0h_device* dev, char* host_name, size_t name_bytes, int* compute_units);
/* ComputeDevice.AllocShared<T>(count) (LlmModel.cs:49-53): device memory, not zeroed. */
int l0h_alloc(l0h_device* dev, size_t bytes, void** out);
/* SharedBuffer<T>.Dispose. */
int l0h_free(l0h_device* dev, void* ptr);
/* SharedBuffer<T>.Write (LlmModel.cs:414, LlmDecoderLayer.cs:320): host -> device, visible to later operations. */
int l0h_write(l0h_device* dev, void* dst, size_t dst_offset_bytes, const void* host_src, size_t bytes);
/* SharedBuffer<T>.ToArray (LlmModel.cs:250, :443): waits for queued work, device -> host. */
int l0h_read(l0h_device* dev, const void* src, size_t src_offset_bytes, void* host_dst, size_t bytes);
/* Fill bytes (LlmKvCache.cs:30-31 zeroes its caches with Write(new float[count])). */
int l0h_fill_zero(l0h_device* dev, void* dst, size_t bytes);
/* ComputeDevice.BeginRecording (LlmModel.cs:353-356, :417-421). */
int l0h_begin_recording(l0h_device* dev);
/* ComputeDevice.EndRecording (LlmModel.cs:380-383, :439-442): submit the recorded list and wait. */
int l0h_end_recording(l0h_device* dev);
/* ComputeDevice.AbortRecording (LlmModel.cs:372-377, :431-437). */
int l0h_abort_recording(l0h_device* dev);
/* Launches the command list of the last l0h_end_recording again, `count` times back to back on
 * the device's stream, and reports the mean HIP-event time of one replay in milliseconds (the
 * reference re-records a list per token, LlmModel.cs:417-443; replaying one is the same work
 * without the recording). L0H_ERR_INVALID_OP when nothing has been recorded, or when memory the
 * recording may use was freed or moved since (l0h_free, workspace or scratch growth). */
int l0h_replay_recording(l0h_device* dev, int count, float* ms_per_replay);
/* Measurement aid, no counterpart in the reference: the kernel launches (graph nodes) of the last
 * recording. */
int l0h_recording_launches(l0h_device* dev, int* launches);
/* ComputeDevice.IsRecording (LlmModel.cs:353, :417). */
int l0h_is_recording(l0h_device* dev, int* out);
/* Wait for every queued operation. */
int l0h_synchronize(l0h_device* dev);
/* Measurement aid, no counterpart in the reference: the HBM read rate of this device in GB/s, from a
 * streaming-read kernel (16-byte non-temporal loads) over a freshly allocated `bytes`-byte buffer
 * (well above the 256 MB Infinity Cache for a cold figure), best of three launch shapes, `reps`
 * launches each. It allocates and frees its buffer. */
int l0h_device_read_bandwidth(l0h_device* dev, size_t bytes, int reps, double* gbs);
/* Message of the calling thread's last failure ("" if none). */
const char* l0h_last_error(void);

/* ======================================================================
 * LlmKernelSuite operators, reference-shaped (fp32 activations)
 * ==================================================================== */

/* LlmGemvKernel.Supports(N) (LlmMatrix.cs:52, :136): N % 4 == 0. */
int l0h_gemv_supports(int out_dim);
/* LlmGemvKernel.MaxRows (LlmDecoderLayer.cs:111): rows per ExecuteRows call. */
int l0h_gemv_max_rows(void);
/* LlmGemvQ8Kernel.Supports(N, K) (LlmMatrix.cs:89): N % 4 == 0 and K % 32 == 0. */
int l0h_gemv_q8_supports(int out_dim, int in_dim);

/* Gemv.Execute(dev, outDim, inDim, x, W, y) (LlmMatrix.cs:134, :138): y[N] = x[K] * W,
 * W in the reference's [K, N] layout, w_dtype L0H_F32 or L0H_F16. */
int l0h_gemv_execute(l0h_device* dev, int out_dim, int in_dim, const float* x, const void* w,
                     int w_dtype, float* y);
/* Gemv.ExecuteRows(dev, rows, outDim, inDim, x, W, y) (LlmMatrix.cs:161, :165). */
int l0h_gemv_execute_rows(l0h_device* dev, int rows, int out_dim, int in_dim, const float* x,
                          const void* w, int w_dtype, float* y);
/* Gemm.Execute(dev, M, N, K, x, W, y) (LlmMatrix.cs:142, :169): fp32 [M,K] x [K,N]. */
int l0h_gemm_execute(l0h_device* dev, int m, int n, int k, const float* x, const float* w,
                     float* y);
/* LlmGemvQ8Kernel.GroupSize (LlmMatrix.cs:29-31; LlmModel.cs:142): 32, the K granularity of the
 * int8 path (Supports asks K % 32 == 0; the activation scratch rounds its width up to it). */
int l0h_gemv_q8_group_size(void);
/* LlmKernelSuite.EnsureQ8Scratch(device, rows, cols) (LlmModel.cs:139-144): the device's int8
 * activation scratch of at least rows x cols fp32 values. Must run before recording starts when it
 * has to grow (L0H_ERR_INVALID_OP inside a recording). */
int l0h_q8_scratch_ensure(l0h_device* dev, int rows, int cols);
/* LlmKernelSuite.Q8Scratch and its RowCapacity (LlmMatrix.cs:242-251): the scratch pointer (NULL
 * before l0h_q8_scratch_ensure), its rows and its columns. */
int l0h_q8_scratch(l0h_device* dev, float** scratch, int* row_capacity, int* cols);
/* GemvQ8.Quantize(dev, rows, inDim, x, scratch) (LlmMatrix.cs:129, :156, :201): stages rows x inDim
 * activations in the scratch for the following Execute calls. The weight-only int8 format keeps
 * activations in fp32, so staging is a copy (the reference quantizes them to int8 here).
 * L0H_ERR_INVALID_OP when the device's own scratch is too small (RequireScratch, :244-251). */
int l0h_gemv_q8_quantize(l0h_device* dev, int rows, int in_dim, const float* x, float* scratch);
/* GemvQ8.Execute(dev, outDim, inDim, scratch, words, scales, y) (LlmMatrix.cs:130, :235): y[N] =
 * (W[N, K] . scratch[K]) * scales[N]. words: int8 [N, K] row-major (four weights per 32-bit word,
 * little-endian, as l0h_quantize_i8pc writes them); scales: fp16 [N], one per output row. */
int l0h_gemv_q8_execute(l0h_device* dev, int out_dim, int in_dim, const float* scratch, const int8_t* w,
                        const uint16_t* scales, float* y);
/* GemvQ8.ExecuteRows(dev, rows, outDim, inDim, scratch, words, scales, y) (LlmMatrix.cs:157, :239):
 * the same for `rows` staged rows, W read once per group of up to 8 rows. */
int l0h_gemv_q8_execute_rows(l0h_device* dev, int rows, int out_dim, int in_dim, const float* scratch,
                             const int8_t* w, const uint16_t* scales, float* y);

/* RMSNorm.Execute(dev, x, residual, w, out, eps, n, rows, addResidual)
 * (LlmDecoderLayer.cs:167, :183-184; LlmModel.cs:394). residual may be NULL when add_residual is 0. */
int l0h_rmsnorm_execute(l0h_device* dev, float* x, const float* residual, const float* w,
                        float* out, float eps, int n, int rows, int add_residual);
/* SwiGLU.Execute(dev, gate, up, n) (LlmDecoderLayer.cs:189). */
int l0h_swiglu_execute(l0h_device* dev, float* gate, const float* up, int n);
/* Add.Execute(dev, a, b, n) (LlmDecoderLayer.cs:194). */
int l0h_add_execute(l0h_device* dev, float* a, const float* b, int n);
/* BiasAdd.Execute(dev, x, bias, n, rows) (LlmDecoderLayer.cs:303-305). */
int l0h_bias_add_execute(l0h_device* dev, float* x, const float* bias, int n, int rows);
/* RoPE.Execute(dev, q, k, positions, headDim, nH, nKv, theta, tokens) (LlmDecoderLayer.cs:415-417). */
int l0h_rope_execute(l0h_device* dev, float* q, float* k, const int* positions, int head_dim,
                     int n_heads, int n_kv_heads, float theta, int tokens);
/* RoPE.ExecuteWithFrequencies(dev, q, k, positions, invFreq, headDim, nH, nKv, attnScale, tokens,
 * rotaryDim) (LlmDecoderLayer.cs:421-423). */
int l0h_rope_execute_with_frequencies(l0h_device* dev, float* q, float* k, const int* positions,
                                      const float* inv_freq, int head_dim, int n_heads,
                                      int n_kv_heads, float attn_scale, int tokens,
                                      int rotary_dim);
/* KvCacheStore.Execute(dev, k, v, K$, V$, pos, kvDim) (LlmDecoderLayer.cs:322).
 * cache_dtype L0H_F32 (the reference's cache, LlmKvCache.cs:21-24) or L0H_F16. */
int l0h_kv_cache_store_execute(l0h_device* dev, const float* k, const float* v, void* k_cache,
                               void* v_cache, int cache_dtype, int pos, int kv_dim);
/* KvCacheStore.ExecuteRows(dev, k, v, K$, V$, pos0, kvDim, tokens) (LlmDecoderLayer.cs:368). */
int l0h_kv_cache_store_execute_rows(l0h_device* dev, const float* k, const float* v,
                                    void* k_cache, void* v_cache, int cache_dtype, int pos0,
                                    int kv_dim, int tokens);
/* Sizes the device's split-reduction workspace for decode attention at this shape, before a
 * recording starts (the attention counterpart of EnsureQ8Scratch, LlmModel.cs:139-144). Attention
 * recorded without it still runs: with as many sequence splits as the workspace holds. */
int l0h_attention_reserve(l0h_device* dev, int batch, int n_heads, int n_kv_heads, int head_dim,
                          int max_seq_len);
/* Attention.Execute(dev, q, K$, V$, out, headDim, nH, nKv, seqLen, maxSeqLen)
 * (LlmDecoderLayer.cs:325-327). Split-K over the sequence: no 15,000-token limit. */
int l0h_attention_execute(l0h_device* dev, const float* q, const void* k_cache,
                          const void* v_cache, int cache_dtype, float* out, int head_dim,
                          int n_heads, int n_kv_heads, int seq_len, int max_seq_len);
/* Attention.ExecutePrefill(dev, q, K$, V$, out, headDim, nH, nKv, pos0, tokens, maxSeqLen)
 * (LlmDecoderLayer.cs:369-371): causal within the chunk, plus every cached slot before it. */
int l0h_attention_execute_prefill(l0h_device* dev, const float* q, const void* k_cache,
                                  const void* v_cache, int cache_dtype, float* out, int head_dim,
                                  int n_heads, int n_kv_heads, int pos0, int tokens,
                                  int max_seq_len);
/* Embedding.Execute(dev, ids, table, out, h, n) (LlmModel.cs:360, :424). */
int l0h_embedding_execute(l0h_device* dev, const int* ids, const float* table, float* out, int h,
                          int n);
/* Copy.Execute(dev, src, dst, srcOffset, n) (LlmModel.cs:368). */
int l0h_copy_execute(l0h_device* dev, const float* src, float* dst, int src_offset, int n);
/* Sampling.Execute(dev, logits, sampled, temperature, randomVal, vocab) (LlmModel.cs:398): greedy
 * argmax, first maximal index (LlmAbstractions.cs:79-92). temperature > 0 is L0H_ERR_UNSUPPORTED. */
int l0h_sampling_execute(l0h_device* dev, const float* logits, int* sampled, float temperature,
                         float random_val, int vocab);

/* ======================================================================
 * Weight-streaming kernels in the [N, K] weight formats (HuggingFace [N, K]
 * weight layout; the role of Gemv / GemvQ8 / Gemm in LlmMatrix.cs:122-218)
 * ==================================================================== */

/* y[r, n] = sum_k x[r, k] * W[n, k] (* scales[n] for L0H_I8PC), fp32 accumulation.
 * w_dtype: L0H_I8PC, L0H_F16, L0H_BF16 or L0H_F32; x_dtype and y_dtype: L0H_F32, L0H_F16 or
 * L0H_BF16. rows 1 is the decode GEMV (LlmMatrix.Project, :122); rows > 1 reads W once per
 * group of rows (LlmMatrix.ProjectRows, :149). */
int l0h_gemv_nk(l0h_device* dev, int w_dtype, int rows, int out_dim, int in_dim, const void* x,
                int x_dtype, const void* w, const uint16_t* scales, void* y, int y_dtype);
/* Prefill GEMM on MFMA: Y[M, N] = X[M, K] * W[N, K]^T, X and W both L0H_F16 or both L0H_BF16,
 * fp32 accumulation, y_dtype L0H_F32, L0H_F16 or L0H_BF16. Replaces the row-chunked
 * ProjectRows of LlmMatrix.cs:149-171 for M >= 64. */
int l0h_gemm_nk(l0h_device* dev, int dtype, int m, int n, int k, const void* x, const void* w,
                void* y, int y_dtype);
/* Prefill GEMM on MFMA with int8 weight-only per-row weights (the chunked-prefill role of
 * LlmMatrix.ProjectRows, LlmMatrix.cs:149-171, for Int8 storage): Y[M, N] = (X[M, K] *
 * W[N, K]^T) * scales[n], X L0H_F16, W int8, scales fp16, fp32 accumulation, y_dtype L0H_F32,
 * L0H_F16 or L0H_BF16. K must be a multiple of 32. */
int l0h_gemm_nk_i8pc(l0h_device* dev, int m, int n, int k, const void* x, const int8_t* w,
                     const uint16_t* scales, void* y, int y_dtype);
/* Batched GQA decode attention (Attention.Execute generalised to a batch; LlmDecoderLayer.cs:325-327).
 * q: [batch, n_heads*head_dim] (q_dtype L0H_F32 or L0H_F16); caches: [batch, max_seq_len,
 * n_kv_heads*head_dim] of cache_dtype; out: [batch, n_heads*head_dim] of out_dtype. Each
 * sequence attends to its slots 0 .. seq_len-1. */
int l0h_attention_decode(l0h_device* dev, const void* q, int q_dtype, const void* k_cache,
                         const void* v_cache, int cache_dtype, void* out, int out_dtype, int batch,
                         int head_dim, int n_heads, int n_kv_heads, int seq_len, int max_seq_len);

/* l0h_attention_decode without any allocation: no counterpart in the reference. For callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, hosts that
 * forbid hipMalloc). Same arguments, kernels and split count as l0h_attention_decode outside a
 * recording; the split partials live in a 4 MiB static device array that each GPU holds until the
 * process ends. L0H_ERR_INVALID_ARG when a shape needs more partials than that (only batch x
 * n_kv_heads in the hundreds with 8 q heads per kv head come close). Calls that overlap on one GPU
 * (other streams, other threads) share the array and race. */
int l0h_attention_decode_noalloc(l0h_device* dev, const void* q, int q_dtype, const void* k_cache,
                                 const void* v_cache, int cache_dtype, void* out, int out_dtype, int batch,
                                 int head_dim, int n_heads, int n_kv_heads, int seq_len, int max_seq_len);

/* ======================================================================
 * Host-side helpers (CPU, no device needed)
 * ==================================================================== */

/* LlmMatrix.FitsInHalf (LlmMatrix.cs:110-120): 1 if every value is finite and |v| <= 65000. */
int l0h_fits_in_half(const float* host_values, size_t count);
/* LlmLayerWeights.Transpose (LlmLayerWeights.cs:226-255): [rows, cols] -> [cols, rows]. */
int l0h_transpose(const float* host_src, int rows, int cols, float* host_dst);
/* Per-output-channel int8 quantization of a HuggingFace [N, K] tensor (role of
 * LlmQ8Quantizer.QuantizeOutIn, LlmMatrix.cs:92): scale = half(max|w| / 127),
 * q = clamp(rint(w / scale), -127, 127). */
int l0h_quantize_i8pc(const float* host_w, int out_dim, int in_dim, int8_t* host_q,
                      uint16_t* host_scales);
/* RopeFrequencies.Compute (RopeFrequencies.cs:60-183). rope_type 0 default, 1 linear, 2 yarn,
 * 3 llama3; negative optional values mean "absent". */
int l0h_rope_frequencies(int head_dim, double theta, int max_position_embeddings, int rope_type,
                         double factor, int original_max_position_embeddings, double beta_fast,
                         double beta_slow, double mscale, double mscale_all_dim,
                         double attention_factor, double low_freq_factor,
                         double high_freq_factor, int truncate, float* host_inv_freq,
                         float* host_attention_factor);

/* ======================================================================
 * LlmMatrix (LlmMatrix.cs:7-260): one projection resident on the device.
 * Device layout is [out, in] (HuggingFace order) for every storage type.
 * ==================================================================== */

/* LlmMatrix.Upload(device, data, inDim, outDim, half) (LlmMatrix.cs:44-57): host data is [in, out]. */
int l0h_matrix_upload(l0h_device* dev, const float* host_in_out, int in_dim, int out_dim,
                      int half, l0h_matrix** out);
/* LlmMatrix.FromHuggingFace(device, hf, sixteenBitSource, name, outDim, inDim, precision)
 * (LlmMatrix.cs:80-106): host hf is [out, in]. L0H_ERR_INVALID_DATA for Float16 values that do
 * not fit a half. */
int l0h_matrix_from_hf(l0h_device* dev, const float* host_out_in, int sixteen_bit_source,
                       int out_dim, int in_dim, int precision, l0h_matrix** out);
/* InDim, OutDim, storage type (L0H_F32/F16/BF16/I8PC), SizeInBytes (LlmMatrix.cs:22-33). */
int l0h_matrix_info(const l0h_matrix* m, int* in_dim, int* out_dim, int* storage,
                    long long* size_in_bytes);
/* Device pointers of the stored weights (and scales for L0H_I8PC, else NULL). */
int l0h_matrix_data(const l0h_matrix* m, const void** w, const uint16_t** scales);
/* LlmMatrix.Project (LlmMatrix.cs:122-144): y[out] = x[in] * W. */
int l0h_matrix_project(l0h_device* dev, const l0h_matrix* m, const float* x, float* y);
/* LlmMatrix.ProjectRows (LlmMatrix.cs:149-171). */
int l0h_matrix_project_rows(l0h_device* dev, const l0h_matrix* m, int rows, const float* x,
                            float* y);
/* LlmMatrix.ProjectAny (LlmMatrix.cs:220-230). */
int l0h_matrix_project_any(l0h_device* dev, const l0h_matrix* m, int rows, const float* x,
                           float* y);
/* LlmMatrix.ProjectShared (LlmMatrix.cs:177-218): 2 to 4 projections of the same x. */
int l0h_matrix_project_shared(l0h_device* dev, int rows, const float* x, int count,
                              const l0h_matrix* const* matrices, float* const* ys);
/* LlmMatrix.Dispose (LlmMatrix.cs:254-260). */
int l0h_matrix_destroy(l0h_matrix* m);

/* ======================================================================
 * Checkpoint ingest (SafetensorsReader.cs, SafetensorsCheckpoint.cs; host)
 * ==================================================================== */

typedef struct l0h_safetensors l0h_safetensors;

/* Element types, in SafetensorsDType order (SafetensorsReader.cs:10-25). */
#define L0H_ST_BOOL 0
#define L0H_ST_U8 1
#define L0H_ST_I8 2
#define L0H_ST_I16 3
#define L0H_ST_U16 4
#define L0H_ST_F16 5
#define L0H_ST_BF16 6
#define L0H_ST_I32 7
#define L0H_ST_U32 8
#define L0H_ST_F32 9
#define L0H_ST_F64 10
#define L0H_ST_I64 11
#define L0H_ST_U64 12

/* SafetensorsCheckpoint.Open (SafetensorsCheckpoint.cs:41-70): a .safetensors file, or a
 * directory holding model.safetensors.index.json and its shards, else model.safetensors. Every
 * header is validated as SafetensorsReader.Open does (SafetensorsReader.cs:110-160, :300-430):
 * L0H_ERR_INVALID_DATA for a malformed file, an index that disagrees with its shards or a tensor
 * in two shards, L0H_ERR_UNSUPPORTED for an unknown dtype. */
int l0h_safetensors_open(const char* path, l0h_safetensors** out);
/* SafetensorsCheckpoint.Dispose. */
int l0h_safetensors_close(l0h_safetensors* st);
/* Number of tensors (SafetensorsCheckpoint.Count). */
int l0h_safetensors_count(const l0h_safetensors* st, int* count);
/* Tensor `index` in name order (SafetensorsTensorInfo): name, L0H_ST_* dtype, rank and the
 * first max_rank dimensions; any output may be null. */
int l0h_safetensors_info(const l0h_safetensors* st, int index, char* name, size_t name_bytes,
                         int* dtype, int* rank, long long* shape, int max_rank);
/* Index of `name`, or -1 when absent (SafetensorsCheckpoint.Contains). */
int l0h_safetensors_find(const l0h_safetensors* st, const char* name, int* index);
/* SafetensorsReader.ReadFloat32 (SafetensorsReader.cs:188-235): an F32, F16, BF16 or F64 tensor
 * as fp32; count must equal its element count. */
int l0h_safetensors_read_f32(const l0h_safetensors* st, const char* name, float* host_dst,
                             size_t count);

/* ======================================================================
 * LlmModel + LlmDecoderLayer (LlmModel.cs, LlmDecoderLayer.cs): a
 * Llama/Qwen2-style decoder resident on the device.
 * ==================================================================== */

/* The HfModelConfig fields the path uses (HfModelConfig.cs:10-120). */
typedef struct {
    int hidden_size;
    int intermediate_size;
    int num_layers;
    int num_attention_heads;
    int num_key_value_heads;
    int head_dim;
    int vocab_size;
    int max_position_embeddings;
    float rms_norm_eps;
    double rope_theta;
    int attention_bias;     /* Qwen2 q/k/v bias (HfModelConfig.cs:186) */
    int tie_word_embeddings; /* lm_head shares the embedding (LlmModel.cs:62) */
    /* rope_scaling (HfRopeScaling, RopeFrequencies.cs:6-40); rope_type 0 means none. */
    int rope_type;
    double rope_factor;
    int rope_original_max_position_embeddings;
    double rope_beta_fast, rope_beta_slow;
    double rope_mscale, rope_mscale_all_dim, rope_attention_factor;
    double rope_low_freq_factor, rope_high_freq_factor;
    int rope_truncate;
} l0h_model_config;

/* Allocates an empty model (LlmModel ctor, LlmModel.cs:34-87): weights must then be set with
 * l0h_model_init_random or l0h_model_set_tensor. precision as LlmWeightPrecision (Auto means
 * Int8, as LlmModel.Load does when int8 kernels exist, :131-134); cache_dtype L0H_F32 or L0H_F16;
 * max_seq_len is the KV cache length (LlmModel.Load, :109-120). */
int l0h_model_create(l0h_device* dev, const l0h_model_config* cfg, int precision, int cache_dtype,
                     int max_seq_len, l0h_model** out);
/* Random-init weights on the device: every projection and the embedding ~ N(0, std^2) from a
 * counter-based generator keyed by seed, then stored at the model's precision; norm weights 1,
 * biases 0. */
int l0h_model_init_random(l0h_model* model, uint64_t seed, float std);
/* Sets one tensor from host fp32 data in HuggingFace naming and layout, e.g.
 * "model.layers.3.self_attn.q_proj.weight" [out, in], "model.norm.weight", "lm_head.weight"
 * (LlmLayerWeights.Load, LlmLayerWeights.cs:110-212; LlmModel.cs:55-63). sixteen_bit_source
 * follows LlmMatrix.FromHuggingFace's rule for Auto precision. */
int l0h_model_set_tensor(l0h_model* model, const char* name, const float* host_data,
                         size_t count, int sixteen_bit_source);
/* LlmModel.Load's weight pass (LlmLayerWeights.Load, LlmLayerWeights.cs:110-212; LlmModel.cs:
 * 55-63): every tensor the config needs, read from the checkpoint as fp32 and stored by
 * l0h_model_set_tensor (F16 / BF16 sources flagged as 16-bit). lm_head.weight is not read when
 * the embeddings are tied. L0H_ERR_INVALID_DATA when a tensor is missing or its shape is not the
 * config's. *loaded (may be null) receives the number of tensors read. */
int l0h_model_load_safetensors(l0h_model* model, const l0h_safetensors* st, int* loaded);
/* Reads back a projection as stored, in HuggingFace [out, in] order: storage type, weights
 * (out*in elements of the storage type: int8 / fp16 / bf16 / fp32) and, for int8, fp16 scales. */
int l0h_model_export_matrix(l0h_model* model, const char* name, int* storage, int* out_dim,
                            int* in_dim, void* host_w, uint16_t* host_scales);
/* Reads a fp32 vector tensor ("model.norm.weight", "...input_layernorm.weight", biases) or the
 * embedding ("model.embed_tokens.weight"). */
int l0h_model_export_vector(l0h_model* model, const char* name, float* host_dst, size_t count);
/* Device pointers of one layer's K and V caches ([max_seq_len, n_kv*head_dim], cache_dtype). */
int l0h_model_kv_cache(l0h_model* model, int layer, void** k_cache, void** v_cache);
/* Device pointer of the logits buffer [vocab] fp32. */
int l0h_model_logits(l0h_model* model, float** logits);
/* LlmModel.ProjectionBytes (LlmModel.cs:92). */
int l0h_model_projection_bytes(l0h_model* model, long long* bytes);
/* How a decode step runs (no reference counterpart; the reference records one command list per
 * token, LlmModel.cs:402-444): L0H_STEP_GRAPH, the step's kernels captured once as a HIP graph and
 * replayed; L0H_STEP_EAGER, the same kernels enqueued one by one (L0H_EAGER_STEP=1); or
 * L0H_STEP_PERSISTENT, the whole step as one persistent kernel (int8 weights with an fp16 cache;
 * disabled: model creation with L0H_STEP_KERNEL=1 fails with L0H_ERR_UNSUPPORTED). */
#define L0H_STEP_GRAPH 0
#define L0H_STEP_EAGER 1
#define L0H_STEP_PERSISTENT 2
int l0h_model_step_path(l0h_model* model, int* path);
/* Kernel launches in one decode step: the nodes of the step's HIP graph (captured if it was not
 * yet), the same kernels an eager step enqueues. No reference counterpart (the reference counts no
 * launches; LlmDecoderLayer.cs:164-195, :291-334 enqueue about 21 operators per layer). */
int l0h_model_step_launches(l0h_model* model, int* launches);
/* LlmModel.Position (LlmModel.cs:219). */
int l0h_model_position(l0h_model* model, int* position);
/* LlmModel.ResetSequence (LlmModel.cs:221). */
int l0h_model_reset_sequence(l0h_model* model);
/* LlmModel.ComputeLogits(tokenId, position) (LlmModel.cs:199-203): host_logits [vocab]. */
int l0h_model_compute_logits(l0h_model* model, int token, int position, float* host_logits);
/* LlmModel.Prefill(promptIds) (LlmModel.cs:224-239): host_logits may be NULL. */
int l0h_model_prefill(l0h_model* model, const int* host_ids, int count, float* host_logits);
/* LlmModel.Decode(tokenId) (LlmModel.cs:242-251): host_logits may be NULL. */
int l0h_model_decode(l0h_model* model, int token, float* host_logits);
/* LlmModel.GenerateGreedy(promptIds, maxNewTokens, stopTokenIds) (LlmModel.cs:156-193): writes
 * up to max_new tokens to host_out and their count to n_out. */
int l0h_model_generate_greedy(l0h_model* model, const int* host_prompt, int prompt_len,
                              int max_new, const int* host_stop, int n_stop, int* host_out,
                              int* n_out);
/* Greedy decode of `steps` tokens from the current position with the step graph replayed
 * back to back and the sampled token fed back on the device (no host round trip per token);
 * starts from `token` at Position and advances Position. host_out receives the tokens. */
int l0h_model_decode_greedy_device(l0h_model* model, int token, int steps, int* host_out);
/* Kernel kinds of one decode step. */
#define L0H_KERNEL_EMBEDDING 0
#define L0H_KERNEL_QKV 1       /* input RMSNorm + q|k|v GEMV + bias + RoPE + KV store */
#define L0H_KERNEL_ATTENTION 2
#define L0H_KERNEL_O_PROJ 3    /* O GEMV + residual */
#define L0H_KERNEL_GATE_UP 4   /* post-attention RMSNorm + gate|up GEMV + SwiGLU */
#define L0H_KERNEL_DOWN 5      /* down GEMV + residual */
#define L0H_KERNEL_LM_HEAD 6   /* final RMSNorm + lm_head GEMV */
#define L0H_KERNEL_ARGMAX 7

typedef struct {
    int kind;            /* L0H_KERNEL_* */
    int layer;           /* decoder layer, -1 for model-level kernels */
    float microseconds;  /* HIP-event time of the launch on the model's stream */
    double bytes;        /* algorithmic HBM bytes of the launch (weights, scales, activations, cache) */
} l0h_kernel_timing;

/* One decode step of `token` at `position` run eagerly, kernel by kernel, with a HIP event pair
 * around every launch (the eager per-stage mode of LlmDecoderLayer.Probe, LlmDecoderLayer.cs:113-119,
 * LlmModel.cs:415-417). Same kernels and results as the graph step. Writes up to `capacity`
 * entries to host_out and the number of launches to count. */
int l0h_model_profile_step(l0h_model* model, int token, int position, l0h_kernel_timing* host_out,
                           int capacity, int* count);
/* Stage callback of l0h_model_probe_step: `count` fp32 values of stage `stage` of decoder layer
 * `layer`, in host memory that is valid during the call (copy what you keep). */
typedef void (*l0h_probe_fn)(void* user, int layer, const char* stage, const float* values, int count);
/* LlmDecoderLayer.Probe (LlmDecoderLayer.cs:113-119): one decode step of `token` at `position`
 * run eagerly (a probe turns recording off, LlmModel.cs:415-417), calling `probe` after each stage
 * of every layer with the stage's values: "input_norm", "q", "k", "v" (after the bias, before
 * RoPE, in head order), "attn_out" (the output projection), "post_norm", "mlp_out" (the down
 * projection) and "output" (the layer's residual stream), as the reference emits them
 * (LlmDecoderLayer.cs:168-195, :315-317). The step itself runs the fused kernels of the graph step,
 * so the cache rows and the logits (host_logits, may be null) are those of l0h_model_compute_logits;
 * the stages the fused kernels never hold in memory (the norms, q/k/v before RoPE, the two
 * projections before their residual adds) are recomputed from the same inputs by the RMSNorm
 * kernel and by the same GEMVs with a plain store. `probe` may be null. */
int l0h_model_probe_step(l0h_model* model, int token, int position, l0h_probe_fn probe, void* user,
                         float* host_logits);
/* Average duration of one kernel kind of the decode step at `position`: `rounds` passes, each
 * launching the kind for every layer (per-layer kinds) or once, back to back between one HIP
 * event pair, so the event cost is amortised and every layer's weights come from HBM. Reports the
 * microseconds and algorithmic bytes per launch and the launches per step. */
int l0h_model_profile_kernel(l0h_model* model, int kind, int position, int rounds, float* avg_us,
                             double* bytes, int* launches);
/* LlmModel.Dispose (LlmModel.cs:308). */
int l0h_model_destroy(l0h_model* model);

#ifdef __cplusplus
}
#endif
#endif
