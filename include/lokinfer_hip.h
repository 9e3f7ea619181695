/* lokinfer MI355X (gfx950) backend: the C-ABI boundary.
 *
 * Two layers, both plain C: pointers, sizes, a hipStream_t passed as void*, an int status (0 = ok).
 *
 * 1. The kernel registry. It replaces the reference's KernelEntry / KernelArgs / findKernel ABI
 *    (lariaus/lokinfer include/lokinfer/runtime/kernel.h:24-74, src/runtime/registry.cpp:39-77) for the GPU
 *    kernel names of its compiled path. lk_run_kernel takes the reference's argument convention
 *    (kernel.h:3-11): ptrs = operands then outs (device pointers), ints = every operand's dims, every out's
 *    dims, then int attrs in attribute-name order, floats = float attrs in attribute-name order. The
 *    reference's Executable::Impl::execute (src/runtime/executable.cpp:582-653) is the caller it replaces.
 *
 * 2. Typed launchers (lk_hip_*), one per kernel family. The registry entries are thin decoders over these.
 *    Each launcher cites the reference kernel it replaces. All enqueue on `stream` and never synchronise.
 *
 * Workspace: kernels that merge partial results across workgroups (split-key decode attention) take a
 * caller-owned device workspace for the partials and merge them in a second launch on the same stream.
 * Calls that share one workspace must be ordered (one stream).
 */
#ifndef LOKINFER_HIP_H
#define LOKINFER_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lk_kernel lk_kernel;

/* ---- registry (reference: registerBuiltinKernels / findKernel / registeredKernels, kernel.h:68-72) ---- */
int lk_init(void);
int lk_num_kernels(void);
const char* lk_kernel_name_at(int i); /* sorted */
const lk_kernel* lk_find_kernel(const char* name);
int lk_kernel_is_gpu(const lk_kernel* k);
int lk_kernel_arity(const lk_kernel* k, int* num_operands, int* num_outs);
/* Reference: KernelEntry::run(ExecCtx&, const KernelArgs&) (kernel.h:56-66). Nonzero on error; the message
 * (the kernel's ExecCtx::error, prefixed with its name) is in lk_last_error(). */
int lk_run_kernel(const lk_kernel* k, void* const* ptrs, uint32_t num_ptrs, const int64_t* ints, uint32_t num_ints,
                  const double* floats, uint32_t num_floats, void* workspace, uint64_t workspace_bytes,
                  void* stream);
const char* lk_last_error(void);

/* ---- device error record (reference: GpuContext::takeGpuError at sync, src/runtime/executable.cpp:850-852) ----
 * Kernels that find invalid data mid-graph (a position outside the cache, an id out of range, a persistent kernel
 * whose exchange timed out) write a neutral value and record the first error per GPU. lk_take_device_error waits
 * for the current device (hipDeviceSynchronize), returns the recorded code (0: none, -1: the read failed) with its
 * detail (the offending position / id / step), and clears the record. The record belongs to the GPU, not to a call:
 * an error is reported by whichever reader comes next (a synchronised executable call, a host read-back), which may
 * be unrelated to the work that recorded it; creating an executable clears an unread record before its init. */
enum {
  LK_DEVERR_EXCHANGE_TIMEOUT = 1,
  LK_DEVERR_POSITION = 2,
  LK_DEVERR_INDEX = 3,
  LK_DEVERR_DURATIONS = 4,
  LK_DEVERR_AUDIO_ROWS = 5
};
int lk_take_device_error(int64_t* detail);
const char* lk_device_error_message(int code);

/* ---- GEMM / conv (reference: gemm_f32_gpu_mps mps.mm:41-84; gemm_bias[_relu]_f32_gpu kokoro_lc.cpp:460-581;
 *      gemm_steel* kokoro_lc.cpp:391-409; conv1d_lc[_res]_f32_gpu kokoro_lc.cpp:81-109) ---- */
/* out[M, N] = (act(A[M, K] . B + bias) + res) * scale; nt: B given as B^T [N, K]; act 0 none, 1 relu, 2 gelu.
 * workspace (optional, may be NULL): with few output tiles and a long K, K is split across workgroups whose
 * partial tiles (split * M * N floats past the first 64 KiB) a second kernel sums; calls sharing a workspace
 * must be stream-ordered. Every form runs on this library's MFMA kernels; results depend only on the shape. */
int lk_hip_gemm_f32(const float* a, const float* b, const float* bias, const float* res, float* out, int64_t m,
                    int64_t n, int64_t k, int nt, int act, float scale, void* workspace, int64_t workspace_bytes,
                    void* stream);
/* channel-last conv1d: x [L, Ci] (Ci % 16 == 0), w [Co, K, Ci] -> out [Lo, Co] = (conv(pre(x)) + b + res) * scale;
 * pre = optional affine [3, Ci] (mean, scale, beta) then snake(alpha) (pre 1) / leaky(slope) (pre 2). K = 1, stride 1,
 * no padding and no prologue run as lk_hip_gemm_f32's NT form */
int lk_hip_conv1d_lc_f32(const float* x, const float* w, const float* bias, const float* res, float* out, int64_t l,
                         int64_t ci, int64_t co, int64_t kw, int stride, int padding, int dilation, float scale,
                         const float* affine, const float* alpha, int pre, float slope, float* stats, void* workspace,
                         int64_t workspace_bytes, void* stream);
/* stats (optional): per-(128-row chunk, channel) (mean, M2) of out, [ceil(Lo / 128), Co, 2], the layout of
 * lk_hip_channel_stats_lc_f32; computed in the conv's epilogue when its tiles are 128 rows, else by a stats pass.
 * workspace (optional, may be NULL): with few output tiles the 16-channel chunks are split over workgroups whose
 * partial tiles (split * Lo * Co floats past the first 64 KiB) a second kernel sums; calls sharing a workspace
 * must be stream-ordered */

/* ---- GEMV (reference: gemv4*_f32_gpu transformer_gpu.cpp:233-251; gemv_rows / gemv1_bias kokoro_lc.cpp:227-267) */
int lk_hip_gemv_f32(const float* x, const float* w, const float* bias, const float* res, float* out, int64_t n,
                    int64_t k, int act, void* workspace, int64_t workspace_bytes, void* stream);
/* workspace (optional, 16-byte aligned): 4 * ceil(K / 64) * N floats of partial sums for the two-launch path;
 * with none (or N % 4 != 0) a single-pass kernel runs. act: 0 none, 2 gelu_tanh. */
int lk_hip_rowdot_f32(const float* mat, const float* vec, const float* bias, int bias_per_row, float* out,
                      int64_t rows, int64_t k, int nvec, int64_t ldo, void* stream);

/* ---- transformer (reference: kokoro_tok.metal:25-204, 465-876; transformer_gpu.cpp:72-222) ---- */
int lk_hip_layernorm_f32(const float* a, const float* bias, const float* r, const float* gamma, const float* beta,
                         float* sum, float* out, int64_t rows, int64_t cols, float eps, int mode, void* stream);
int lk_hip_bias_gelu_f32(const float* x, const float* bias, float* out, int64_t rows, int64_t cols, void* stream);
int lk_hip_attention_qkv_f32(const float* qkv, const float* bias, float* out, int64_t t, int heads, int causal,
                             void* stream);
/* split-key decode attention (waves of 64-key chunks, then a merge launch); pos is a device i64[1]. Up to 8192
 * keys each wave takes one chunk; beyond, each wave takes ceil(chunks / 128) chunks, combined online, so a head
 * has at most 128 partials (workspace: heads * waves * 66 floats, lk_hip_attention_decode_workspace_bytes) */
int64_t lk_hip_attention_decode_workspace_bytes(int heads, int64_t cap);
int lk_hip_attention_decode_f32(const float* qkv, float* kc, float* vc, const int64_t* pos, const float* bias,
                                float* out, int64_t cap, int heads, int64_t max_keys, int write_kv, void* workspace,
                                int64_t workspace_bytes, void* stream);
/* Allocation-free variant of lk_hip_attention_decode_f32 (no counterpart in the reference): for callers that
 * cannot allocate device memory (HIP graph capture of a serving loop, harnesses that forbid hipMalloc). The chunk
 * partials go to a fixed 2 MiB device array the library holds on each GPU for the life of the process
 * (lk_hip_attention_decode_noalloc_max_floats() floats: heads * waves * 66 must fit, waves as above), so it calls no
 * hipMalloc. Returns 4 when the call does not fit. Calls that overlap on one GPU race on that array. */
int64_t lk_hip_attention_decode_noalloc_max_floats(void);
int lk_hip_attention_decode_f32_noalloc(const float* qkv, float* kc, float* vc, const int64_t* pos, const float* bias,
                                        float* out, int64_t cap, int heads, int64_t max_keys, int write_kv,
                                        void* stream);
int lk_hip_kv_write_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias, int64_t d,
                        int64_t cap, void* stream);
/* chunked prefill / generate (reference kv_write_rows_f32_gpu, attention_cache[_sg]_f32_gpu,
 * python/lokinfer/ops/transformer.py:239-268, 348-351; kernels/gpu/kokoro_lc.cpp:887-965): the T rows of qkv sit at
 * positions pos..pos+T-1 (pos a device i64[1]). kv_write_rows writes k, v (+ bias) there (rows >= cap dropped);
 * attention_cache attends query i causally over cache rows 0..pos+i (q bias added, head_dim 64; a query at
 * position >= cap gets NaN). The reference rejects pos + T > cap on the host; here pos lives on the device. */
int lk_hip_kv_write_rows_f32(float* kc, float* vc, const float* qkv, const int64_t* pos, const float* bias,
                             int64_t t, int64_t d, int64_t cap, void* stream);
int lk_hip_attention_cache_f32(const float* qkv, const float* kc, const float* vc, const int64_t* pos,
                               const float* bias, float* out, int64_t t, int heads, int64_t cap, void* stream);
/* split-K partials and their consumer (reference gemm_splitk_f32_gpu / add_bias_layernorm2_sk_f32_gpu,
 * transformer_gpu.cpp:253-320, python/lokinfer/ops/transformer.py:441-472): part[s] = A[:, sK/S:(s+1)K/S] .
 * B[sK/S:(s+1)K/S, :] for s < splits, part f32[S, M, N], K % (16 S) == 0, K and N % 4 == 0, 16-byte aligned;
 * then sum = part[0] + ... + part[S-1] + bias + r, out = LN(sum), cols <= 2048 */
int lk_hip_gemm_splitk_f32(const float* a, const float* b, float* part, int64_t m, int64_t n, int64_t k, int splits,
                           void* stream);
int lk_hip_add_bias_ln_sk_f32(const float* parts, int64_t splits, const float* bias, const float* r,
                              const float* gamma, const float* beta, float* sum, float* out, int64_t rows,
                              int64_t cols, float eps, void* stream);

/* ---- fused batch-1 decode layer (backend ops; one layer's reference sequence gemv4*_f32_gpu ->
 * attention_decode_split_f32_gpu -> gemv4 -> add_bias_layernorm2_f32_gpu, transformer_gpu.cpp:122-251,
 * kokoro_tok.metal:36-117, in 5 launches instead of 13). GEMVs write row-slice partial sums part[S, N]
 * (S = lk_hip_gemv_partial_slices(K)); the consumer reduces the slices in order. */
int64_t lk_hip_gemv_partial_slices(int64_t k);
/* xmode 0: x is a vector [K]; 1: x = gelu_tanh(sum of xpart[xslices, K] + xbias); 2: x = merge of decode
 * chunk partials xpart[K / 64, chunks, 66]; 3: sum = (slices of xpart) + xbias + res is written to sum_out and
 * x = LayerNorm(sum; gamma, beta, eps) (K <= 1024; xpart / xbias may be null). N % 4 == 0. */
int lk_hip_gemv_partial_f32(int xmode, const float* x, const float* xpart, const float* xbias, int64_t xslices,
                            int chunks, const float* res, const float* gamma, const float* beta, float* sum_out,
                            float eps, const float* w, float* part, int64_t n, int64_t k, void* stream);
/* q, k, v = slice sums of qkv_part[slices, 3D] + bias; writes row pos of kc / vc and the per-(head, 64-key
 * chunk) partials chunk_part[heads, ceil(cap / 64), 66] = (max, sum, acc[64]); an invalid pos writes NaN. */
int lk_hip_attention_decode_part_f32(const float* qkv_part, int64_t slices, float* kc, float* vc, const int64_t* pos,
                                     const float* bias, float* chunk_part, int64_t cap, int heads, void* stream);
/* Layer-0 variant of xmode 3 whose sum is two embedding rows: sum = table[id[0]] + table2[id2[0]] (the GPT-2
 * token + position lookups, which the reference does on the host, models/gpt2.py:189-190), written to sum_out;
 * x = LayerNorm(sum). An id out of range records LK_DEVERR_INDEX and yields NaN. K <= 1024, K % 4 == 0. */
int lk_hip_gemv_partial_embed_ln_f32(const float* table, const int64_t* id, const float* table2, const int64_t* id2,
                                     int64_t rows, int64_t rows2, const float* gamma, const float* beta, float eps,
                                     const float* w, float* part, float* sum_out, int64_t n, int64_t k, void* stream);
/* Tied LM head + final LayerNorm + greedy argmax of a decode step (replaces add_bias_layernorm2_f32_gpu,
 * gemm_nt_f32_gpu_mps and the Python argmax, models/gpt2.py:225, 243, 349-355): logits[r] = LayerNorm((slices of
 * part) + bias + res) . table[r, :], argmax[0] = first index of the max logit. Two launches; workspace >= 16
 * min(512, ceil(rows / 4)) bytes (3 when short). K <= 1024, K % 4 == 0. */
int lk_hip_lm_head_ln_argmax_f32(const float* part, int64_t slices, const float* bias, const float* res,
                                 const float* gamma, const float* beta, float eps, const float* table, float* logits,
                                 int64_t* argmax, int64_t rows, int64_t k, void* workspace, int64_t workspaceBytes,
                                 void* stream);
/* sum = (slices of part[slices, N]) + bias + res; ln = LayerNorm(sum); one workgroup, N <= 1024 */
int lk_hip_reduce_ln_f32(const float* part, int64_t slices, const float* bias, const float* res, const float* gamma,
                         const float* beta, float* sum_out, float* ln_out, int64_t n, float eps, void* stream);

/* ---- Kokoro frame-rate, channel-last (reference: kokoro_lc.metal:143-398) ---- */
int lk_hip_channel_stats_lc_f32(const float* x, float* stats, int64_t l, int64_t c, void* stream);
int lk_hip_adain_affine_lc_f32(const float* stats, const float* gb, float* affine, int64_t l, int64_t c,
                               int64_t creal, float eps, void* stream);
int lk_hip_act_lc_f32(const float* x, const float* affine, const float* alpha, float* out, int64_t l, int64_t c,
                      int act, float slope, void* stream);
int lk_hip_convt_gather_lc_f32(const float* y, const float* bias, const float* add, float* out, int64_t lin,
                               int64_t lout, int64_t co, int k, int stride, int pad, int reflect_left, void* stream);
int lk_hip_dwconvt_lc_f32(const float* x, const float* w, const float* bias, float* out, int64_t lin, int64_t lout,
                          int64_t c, int k, int stride, int pad, void* stream);
int lk_hip_upsample2_lc_f32(const float* x, float* out, int64_t l, int64_t c, void* stream);
int lk_hip_concat_pad_lc_f32(const float* a, const float* b, float* out, int64_t l, int64_t ca, int64_t cb,
                             int64_t cout, void* stream);
int lk_hip_transpose_f32(const float* x, float* out, int64_t r, int64_t c, int64_t ldx, void* stream);
int lk_hip_elementwise_f32(const float* a, const float* b, const float* c, float* out, int64_t n, int op, float s,
                           void* stream);
int lk_hip_istft_lc_f32(const float* x, float* out, int64_t l, int64_t cpad, int nfft, int hop, void* stream);

/* ---- token-rate front end on the device (reference: host kernels embedding_f32_cpu kernels/cpu/kokoro_norm.cpp,
 *      GPT-2 argmax in Python models/gpt2.py:348-359) ---- */
int lk_hip_embedding_f32(const float* table, const int64_t* ids, const float* table2, const int64_t* ids2, float* out,
                         int64_t n, int64_t d, int64_t rows, int64_t rows2, void* stream);
/* out[i] = pos[0] + i (reference host kernel arange_offset_i64_cpu, kernels/cpu/decode.cpp:221) */
int lk_hip_arange_offset_i64(const int64_t* pos, int64_t* out, int64_t n, void* stream);
/* out[0] = indices[i] of the largest values[i] (ties: the smallest index), i < n: the last pass of an argmax whose
 * first pass left (value, index) pairs */
int lk_hip_argmax_pairs_f32(const float* values, const int64_t* indices, int64_t* out, int64_t n, void* stream);
int lk_hip_argmax_f32(const float* x, int64_t* out, int64_t rows, int64_t n, void* workspace,
                      int64_t workspace_bytes, void* stream);

/* ---- Kokoro token-rate sequence kernels (reference host kernels: lstm_bidir[_t]_f32_cpu ops/kokoro.py:88-116,
 *      repeat_interleave_f32_cpu kokoro_misc.cpp:253-265, adalayernorm_f32_cpu kokoro_norm.cpp:10-62,
 *      concat_cols / broadcast_rows ops/kokoro.py:141-173) ---- */
/* x [T, I], w_ih [8H, I], w_hh_t [H, 8H] (W_hh^T), b [8H] = b_ih + b_hh -> out [T, 2H]; workspace >= T * 8H floats */
int lk_hip_lstm_bidir_f32(const float* x, const float* w_ih, const float* w_hh_t, const float* b, float* out,
                          int64_t t, int64_t in, int64_t h, void* workspace, int64_t workspace_bytes, void* stream);
/* Two lk_hip_lstm_bidir_f32 of the same length T (H = 256) in one recurrence launch (MI355X backend; no reference
 * counterpart: the Kokoro graph runs its text encoder's BiLSTM beside the duration encoder's first). Workspace:
 * 2 (ceil256(T 8H 4) + 8384) bytes. */
int lk_hip_lstm_bidir2_f32(const float* x1, const float* wih1, const float* whhT1, const float* b1, float* out1,
                           int64_t in1, const float* x2, const float* wih2, const float* whhT2, const float* b2,
                           float* out2, int64_t in2, int64_t t, int64_t h, void* workspace, int64_t workspaceBytes,
                           void* stream);
int lk_hip_repeat_interleave_f32(const float* x, const int64_t* dur, float* out, int64_t t, int64_t c, int64_t frames,
                                 void* stream);
int lk_hip_adalayernorm_f32(const float* x, const float* gb, float* out, int64_t r, int64_t c, float eps,
                            void* stream);
int lk_hip_concat_bcast_f32(const float* x, const float* v, float* out, int64_t r, int64_t c1, int64_t c2,
                            void* stream);

/* ---- Kokoro signal path (reference host kernels: harmonic_source_f32_cpu kokoro_signal.cpp:89-192,
 *      stft_magphase_f32_cpu kokoro_signal.cpp:196-273, decoder F0_conv / N_conv conv1d_f32_cpu) ---- */
/* f0 [n], noise [300 n, 9], w [9], b [1] -> out [300 n]; workspace >= 9 n floats */
int lk_hip_harmonic_source_f32(const float* f0, const float* noise, const float* w, const float* b, float* out,
                               int64_t n, void* workspace, int64_t workspace_bytes, void* stream);
/* x [S] -> out [S / hop + 1, ldo]: magnitude in columns 0..K-1, phase in K..2K-1 (K = nfft / 2 + 1), rest 0 */
int lk_hip_stft_magphase_lc_f32(const float* x, float* out, int64_t s, int nfft, int hop, int64_t ldo, void* stream);
int lk_hip_conv1d_1ch_f32(const float* x, const float* w, const float* b, float* out, int64_t l, int k, int stride,
                          int pad, void* stream);

/* ---- Winograd / Toom-Cook conv1d (reference: wino_tf*, wino_mm*, wino_adain_affine ops/winograd.py:128-218,
 *      launchers winograd.cpp:73-160). U [A, n Ci, Co] and tr = [BT | AT] come from the host weight transform
 *      (lokinfer_amd/winograd.py wino_weights); A = 6 (K = 3), 4 (K = 3, tile 2), 7 (K = 4..12, n = 2 or 3). ---- */
/* x [L, C] -> V [d, A, rmax, C] (v_rows = d A rmax), of h = x (act 0), snake(affine(x), alpha) (1) or
 * leaky(affine(x), slope) (2); padding % dilation == 0, C % 4 == 0 */
int lk_hip_wino_tf_lc_f32(const float* x, const float* tr, const float* affine, const float* alpha, float* v,
                          int64_t l, int64_t c, int dilation, int padding, int kernel, int tile, int64_t v_rows,
                          int act, float slope, void* stream);
/* out [Lo, Co] = (AT (V_xi U_xi) + bias [+ res]) * scale; Ci % 16 == 0, Co % 64 == 0; stats (optional)
 * [d ceil(ceil(Lo / d) / 128), Co, 2]: (mean, M2) per 128-row chunk of each residue class. workspace
 * (optional, may be NULL): with dilation 1 and a grid too small for the chip, the point-chunk steps are split
 * over up to 8 workgroups whose partial rows (split * Lo * Co floats past the first 64 KiB) a second kernel
 * sums; calls sharing a workspace must be stream-ordered */
int lk_hip_wino_mm_lc_f32(const float* v, const float* u, const float* bias, const float* res, float* out,
                          const float* tr, float* stats, int64_t v_rows, int64_t ci, int64_t co, int64_t lo,
                          int dilation, int groups, int kernel, int tile, float scale, void* workspace,
                          int64_t workspace_bytes, void* stream);
/* The same with U given tiled (MI355X backend; the wino_mm ops' u_layout = 1), ut [A, Co / 64, (Ci / 16) N 4 64 4]:
 * ut[x, cb, (((c N + g) 4 + k4) 64 + j) 4 + q] = U[x, g Ci + 16 c + 4 k4 + q, 64 cb + j] (lokinfer_amd/winograd.py
 * wino_weights_t), each pipeline step's slab of U contiguous in the order the kernel stages it; identical
 * arithmetic, so the same bits as lk_hip_wino_mm_lc_f32. */
int lk_hip_wino_mm_ut_lc_f32(const float* v, const float* ut, const float* bias, const float* res, float* out,
                             const float* tr, float* stats, int64_t v_rows, int64_t ci, int64_t co, int64_t lo,
                             int dilation, int groups, int kernel, int tile, float scale, void* workspace,
                             int64_t workspace_bytes, void* stream);
/* stats [s, c, 2] of a length-row output -> af [3, c] = (mean, (1 + g) / sqrt(var + eps), b), gb [2 creal];
 * channels >= creal get 0 */
int lk_hip_wino_adain_affine_lc_f32(const float* stats, const float* gb, float* af, int64_t s, int64_t c,
                                    int64_t creal, int dilation, int64_t length, float eps, void* stream);

/* ---- f16 language model (Qwen3-ASR LM; reference f16 GPU op family kernels/gpu/f16_gpu.cpp:1011-1050, contracts
 *      python/lokinfer/ops/f16.py, f16_gpu.py). f16 storage (pointers to IEEE half), f32 math and accumulation, one
 *      rounding at each output. Weights of the GEMM-like ops are packed once as W^T f16[N', K]
 *      (lk_hip_f16_transpose); the reference fixes only the math and leaves the layout to the kernel. ---- */
/* out f16[M, N] = x f16[M, K] @ W (+ bias f16[N]) (+ res f16[M, N]), or silu(x @ Wg) * (x @ Wu) with swiglu = 1
 * (W^T rows [gate | up], N' = 2N): gemm[_bias]_f16_gpu, gemm[_bias|_add|_swiglu]_opt_f16_gpu. K % 8 == 0, 16-byte
 * aligned x and W^T. M = 1 runs a GEMV; M > 1 the f16 MFMA tile kernels (f32 accumulation, the epilogue fused).
 * workspace (optional): split-K partials when the grid is small. */
int lk_hip_f16_gemm(const void* x, const void* wt, const void* bias, const void* res, void* out, int64_t m, int64_t n,
                    int64_t k, int swiglu, void* workspace, int64_t workspace_bytes, void* stream);
int64_t lk_hip_f16_gemm_workspace_bytes(int64_t m, int64_t n, int swiglu);
/* rmsnorm_gemm[_swiglu]_opt_f16_gpu: out = rmsnorm(x, g) @ W [swiglu]; ws f16[M, K] receives the normalized rows
 * when M > 1 (unused at M = 1, where the GEMV normalizes the row itself) */
int lk_hip_f16_rms_gemm(const void* x, const void* g, const void* wt, void* out, void* ws, int64_t m, int64_t n,
                        int64_t k, float eps, int swiglu, void* workspace, int64_t workspace_bytes, void* stream);
/* lm_head_last[_opt]_f16_gpu: out f32[1, V] = x[T-1] . table f16[V, D]^T */
int lk_hip_f16_lm_head(const void* x, const void* table, float* out, int64_t t, int64_t d, int64_t v, void* stream);
/* rmsnorm[_heads]_f16_gpu: groups of `width` values of x f16[rows, C] (width = C, or the head width) */
int lk_hip_f16_rmsnorm(const void* x, const void* g, void* out, int64_t rows, int64_t c, int64_t width, float eps,
                       void* stream);
/* rope_f16_gpu: rotate_half RoPE per 128-wide head at positions pos + i (pos a device i64[1]) */
int lk_hip_f16_rope(const void* x, const int64_t* pos, void* out, int64_t t, int64_t c, float theta, void* stream);
/* qknorm_rope_kv_opt_f16_gpu: qkv f16[T, 128 (qh + 2 kvh)] -> q f16[T, 128 qh]; k, v to cache rows pos.. */
int lk_hip_f16_qknorm_rope_kv(const void* qkv, const void* qg, const void* kg, const int64_t* pos, void* kc, void* vc,
                              void* q, int64_t t, int qh, int kvh, int64_t cap, float eps, float theta, void* stream);
/* attention_gqa[_opt]_f16_gpu: causal GQA of q f16[T, 128 qh] over the caches f16[cap, 128 kvh]; T = 1 needs
 * lk_hip_f16_attention_workspace_bytes of workspace (returns 3 when short) */
int64_t lk_hip_f16_attention_workspace_bytes(int qh, int64_t cap);
int lk_hip_f16_attention_gqa(const void* q, const void* kc, const void* vc, const int64_t* pos, void* out, int64_t t,
                             int qh, int kvh, int64_t cap, void* workspace, int64_t workspace_bytes, void* stream);
/* decode step (T = 1) fusions (backend ops; the reference runs qknorm_rope_kv_opt -> attention_gqa_opt and
 * rmsnorm -> lm_head_last_opt, model.py:393-401, 287-288): attention_decode_qkr_opt_f16_gpu goes from the raw qkv
 * projections f16[1, 128 (qh + 2 kvh)] to the attention output f16[1, 128 qh] in one launch (QK-norm, RoPE, row pos of
 * both caches, key-split chunks (a wave takes ceil(chunks / 128) consecutive 64-key chunks, and two q heads of a kv
 * group on caches of 128 chunks or more), and their merge by the last wave of each head to finish; counters: qh unsigned
 * ints, zero before the first call and left zero; workspace as lk_hip_f16_attention_workspace_bytes, 3 when short);
 * rmsnorm_lm_head_last_opt_f16_gpu normalizes the last row inside the LM-head GEMV. Each equals its composition bit
 * for bit. */
int lk_hip_f16_attention_decode_qkr(const void* qkv, const void* qg, const void* kg, const int64_t* pos, void* kc,
                                    void* vc, void* out, unsigned* counters, int qh, int kvh, int64_t cap, float eps,
                                    float theta, void* workspace, int64_t workspace_bytes, void* stream);
int lk_hip_f16_rms_lm_head(const void* x, const void* g, const void* table, float* out, int64_t t, int64_t d, int64_t v,
                           float eps, void* stream);
/* kv_write_f16_gpu, embedding_f16_gpu, scatter_audio_f16_gpu, add_f16_gpu (op 0), silu_mul_f16_gpu (op 1). A device
 * kernel cannot raise the reference's host errors: rows past the cache are dropped, an id out of range or a pad row
 * without an audio row gives a NaN row. */
int lk_hip_f16_kv_write(void* kc, void* vc, const void* k, const void* v, const int64_t* pos, int64_t t, int64_t d,
                        int64_t cap, void* stream);
int lk_hip_f16_embedding(const int64_t* ids, const void* table, void* out, int64_t t, int64_t vocab, int64_t d,
                         void* stream);
int lk_hip_f16_scatter_audio(const void* x, const int64_t* ids, const void* audio, void* out, int64_t t, int64_t d,
                             int64_t na, int64_t pad_id, void* stream);
int lk_hip_f16_elementwise(const void* a, const void* b, void* out, int64_t n, int op, void* stream);
/* weight packing: W f16[K, N] -> W^T f16[N, K] */
int lk_hip_f16_transpose(const void* w, void* wt, int64_t k, int64_t n, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOKINFER_HIP_H */
