/* libkvpack: the quantized decode kernel pack for MI355X (gfx950).
 *
 * C ABI over hand-written HIP kernels for the three operators of
 * vladmt06/kernelverify's kernel pack:
 *
 *   - affine group-quantized matvec        (kernelverify/pack/wide_qmv.py)
 *   - quantized-KV decode attention         (kernelverify/pack/kv_attention.py)
 *   - top-k MoE routing + gather-qmv        (kernelverify/pack/moe_dispatch.py)
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers owned by the caller; the
 *     library never allocates in a compute call. Scratch space is a caller
 *     buffer whose size a *_workspace_bytes() query returns.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream)
 *     and is stream-ordered; nothing synchronises the host.
 *   - Every function returns an int status: KVP_OK (0) or a negative code.
 *     kvp_last_error() returns the calling thread's last diagnostic.
 *     Argument checks happen before anything is enqueued, so a failed call
 *     has no effect on the device.
 *   - Quantized artefacts use the MLX affine layout the reference reads
 *     (kernelverify/pack/wide_qmv.py:185-201): per row, a contiguous
 *     little-endian bit stream of `bits`-wide codes viewed as uint32 words
 *     (code i at bits [i*bits, (i+1)*bits)), plus fp16 scale and bias per
 *     64-code group; the dequantized value is scale * q + bias.
 *   - fp16 arguments are IEEE binary16 (`void*`, 2 bytes per element).
 *   - Accumulation is binary32 throughout and outputs are rounded to their
 *     storage dtype once (kernelverify/tolerance/contract.py:23-30, C1),
 *     with two stated exceptions where an fp32 intermediate enters the
 *     matrix cores as an fp16 hi + lo pair, about 22 significant bits (the
 *     products are exact, the sums fp32): the probability-scaled value
 *     weight p * scale of kvp_kv_decode's value side at 4 and 8 bits, and
 *     the SwiGLU hidden state entering kvp_moe_swiglu's down projection at
 *     4 and 8 bits. Every other intermediate is binary32 or wider.
 */
#ifndef KVPACK_H_
#define KVPACK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. They map one-to-one onto the runner statuses of
 * kernelverify/runners/result.py:67-74. */
enum {
  KVP_OK = 0,
  KVP_INVALID = -1,      /* bad argument: RunStatus.INVALID_SPEC */
  KVP_UNSUPPORTED = -2,  /* valid request this build does not implement */
  KVP_LAUNCH_ERROR = -3, /* the HIP runtime refused the launch */
  KVP_NO_DEVICE = -4     /* no gfx950 device visible: RunStatus.UNSUPPORTED */
};

/* Output dtypes (the reference's `$T` template hole: half or float). */
enum { KVP_F16 = 1, KVP_F32 = 2 };

/* Library version string, e.g. "kvpack 0.1.0 gfx950". */
const char* kvp_version(void);

/* Copies the calling thread's last diagnostic (NUL-terminated, truncated to
 * `cap`) and returns its full length. Empty after a successful call. */
size_t kvp_last_error(char* buf, size_t cap);

/* Device facts the runner's probe() reports
 * (replaces kernelverify/runners/device.py:123-132 MetalDevice.info).
 * name_cap bytes of the marketing name go to `name`; the rest are counts. */
int kvp_device_info(int device, char* name, size_t name_cap, char* arch, size_t arch_cap,
                    int* compute_units, int* max_threads_per_block,
                    size_t* lds_per_block, size_t* global_mem_bytes, int* clock_khz);

/* ------------------------------------------------------------------------
 * MLX-affine group quantization of fp16 rows into the kernel layout.
 * Replaces canonical_quantize + pack_codes
 * (kernelverify/schemas/quant_contract.py:60-104, pack/wide_qmv.py:185-201)
 * and quantize_cache (kernelverify/pack/kv_attention.py:270-283); bit-exact
 * with the contract's fp32 algorithm.
 *   w      fp16   [rows][cols], cols % 64 == 0
 *   w_q    uint32 [rows][cols * bits / 32]
 *   scales, biases fp16 [rows][cols / 64]
 * bits in {2, 3, 4, 8}.
 * ---------------------------------------------------------------------- */
int kvp_quantize_affine(const void* w, int rows, int cols, int bits, uint32_t* w_q,
                        void* scales, void* biases, void* stream);

/* ------------------------------------------------------------------------
 * Quantized matvec: out[m, r] = sum_k x[m, k] * (scale[r, k/64] * q[r, k]
 *                                                + bias[r, k/64])
 * Replaces the runner-door kernel `kv_wide_qmv`
 * (kernelverify/pack/wide_qmv.py:65-135, bindings :228-260).
 *   x      fp16   [m][d_in]
 *   w_q    uint32 [d_out][d_in * bits / 32]
 *   scales fp16   [d_out][d_in / 64]
 *   biases fp16   [d_out][d_in / 64]
 *   out    fp16 or fp32 (out_dtype) [m][d_out]
 * bits in {2, 3, 4, 8}; 1 <= m <= 16; d_in % 64 == 0; any d_out >= 1.
 * ---------------------------------------------------------------------- */
int kvp_qmv(const void* x, const uint32_t* w_q, const void* scales, const void* biases,
            void* out, int out_dtype, int m, int d_out, int d_in, int bits, void* stream);

/* ------------------------------------------------------------------------
 * Quantized-KV decode attention, one step, split over cached positions
 * with a log-sum-exp combine.
 * Replaces `kv_attn_decode` (kernelverify/pack/kv_attention.py:85-234,
 * bindings :292-352), generalised past its T <= 1024 capacity bound (:77).
 *   q            fp16   [batch][n_heads][head_dim]
 *   k_wq, v_wq   uint32 [C][n_kv_heads][t_stride][head_dim * bits / 32]
 *   k_/v_scales,
 *   k_/v_biases  fp16   [C][n_kv_heads][t_stride][head_dim / 64]
 *                where C = batch when cache_per_sequence != 0, else 1
 *                (C = 1 is the reference's layout: one cache read by every
 *                batch row, :135, :202)
 *   new_k, new_v fp16   [batch][n_kv_heads][head_dim]  (this step's entry,
 *                        used at full precision as position t_cached[b])
 *   t_cached     int32  [batch] device array: cached positions of each
 *                        sequence (read as min(max(t_cached[b], 0), t_stride))
 *   out          fp16 or fp32 [batch][n_heads][head_dim]
 * Query head h reads cache head h / (n_heads / n_kv_heads) (GQA, :99-103).
 * Scores are scaled by 1/sqrt(head_dim). head_dim in {64, 128};
 * bits in {2, 3, 4, 8}; n_heads % n_kv_heads == 0.
 * chunk: cached positions per split (0 = the library's choice); a multiple
 * of 64. workspace: at least kvp_kv_decode_workspace_bytes(...) bytes;
 * calls sharing a workspace must be ordered (one stream).
 * ---------------------------------------------------------------------- */
size_t kvp_kv_decode_workspace_bytes(int batch, int n_heads, int head_dim, int t_stride,
                                     int chunk);
int kvp_kv_decode(const void* q, const uint32_t* k_wq, const void* k_scales,
                  const void* k_biases, const uint32_t* v_wq, const void* v_scales,
                  const void* v_biases, const void* new_k, const void* new_v,
                  const int32_t* t_cached, void* out, int out_dtype, int batch, int n_heads,
                  int n_kv_heads, int head_dim, int t_stride, int bits, int cache_per_sequence,
                  int chunk, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free variant of kvp_kv_decode. No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments and results as kvp_kv_decode without the workspace: the split
 * partials live in a fixed static device array of
 * kvp_kv_decode_static_scratch_bytes() bytes (4 MiB) per GPU, held until the
 * process ends. A call whose kvp_kv_decode_workspace_bytes(...) exceeds that
 * is refused with KVP_INVALID. Nothing is allocated and nothing is cleared:
 * every partial a call reads is written by the same call. Every call on one
 * GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams at once) race; order them on one stream. */
size_t kvp_kv_decode_static_scratch_bytes(void);
int kvp_kv_decode_static(const void* q, const uint32_t* k_wq, const void* k_scales,
                         const void* k_biases, const uint32_t* v_wq, const void* v_scales,
                         const void* v_biases, const void* new_k, const void* new_v,
                         const int32_t* t_cached, void* out, int out_dtype, int batch,
                         int n_heads, int n_kv_heads, int head_dim, int t_stride, int bits,
                         int cache_per_sequence, int chunk, void* stream);

/* ------------------------------------------------------------------------
 * MoE routing: softmax over all n_experts, top-k BY PROBABILITY with ties
 * to the lower expert index, gates renormalised over the k chosen.
 * Replaces `kv_moe_routing` (kernelverify/pack/moe_dispatch.py:39-79,
 * bindings :161-196), generalised from k = 2 to 1 <= k <= 32.
 *   kvp_moe_route:        logits = x @ router^T in fp32 (x fp16 [n][d],
 *                         router fp16 [n_experts][d]), as the reference.
 *   kvp_moe_route_logits: logits given, fp32 [n][n_experts].
 *   idx  uint32 [n][k] (descending probability), gate fp32 [n][k].
 * n_experts <= 1024.
 * ---------------------------------------------------------------------- */
int kvp_moe_route(const void* x, const void* router, uint32_t* idx, float* gate, int n,
                  int d, int n_experts, int k, void* stream);
int kvp_moe_route_logits(const float* logits, uint32_t* idx, float* gate, int n,
                         int n_experts, int k, void* stream);

/* Stable counting sort of the n*k (token, slot) pairs by expert (no
 * reference kernel: the reference dispatches per token, :84-138).
 *   offsets int32 [n_experts + 1]: pairs of expert e are perm[offsets[e] ..
 *           offsets[e+1]); perm int32 [n*k]: flat index token*k + slot,
 *           ascending within each expert. Bit-exact and deterministic.
 * n * k <= 8192 (one workgroup holds the pairs). */
int kvp_moe_permute(const uint32_t* idx, int32_t* offsets, int32_t* perm, int n, int k,
                    int n_experts, void* stream);

/* Single-linear dispatch, the reference's contract at any k:
 *   out[t, r] = sum_s gate[t, s] * (x[t] . dequant(W[idx[t, s]])[r])
 * Replaces `kv_moe_dispatch` (kernelverify/pack/moe_dispatch.py:84-138).
 *   x fp16 [n][d_in]; w_q uint32 [n_experts][d_out][d_in * bits / 32];
 *   scales, biases fp16 [n_experts][d_out][d_in / 64]; out [n][d_out].
 * A slot naming no expert (idx >= n_experts) adds nothing, as in
 * kvp_moe_swiglu. bits in {2, 3, 4, 8}; k <= 32. */
int kvp_moe_dispatch(const void* x, const uint32_t* idx, const float* gate,
                     const uint32_t* w_q, const void* scales, const void* biases, void* out,
                     int out_dtype, int n, int k, int n_experts, int d_out, int d_in, int bits,
                     void* stream);

/* SwiGLU expert MLP over routed tokens (BASELINE's gate/up/down form; no
 * reference counterpart beyond the single-linear contract above):
 *   h_{t,s}  = silu(x_t . Wg_e) * (x_t . Wu_e)      (fp32, e = idx[t, s])
 *   out[t]   = sum_s gate[t, s] * (h_{t,s} . Wd_e)  (slots in order s = 0..k-1)
 * gate_/up_ weights [n_experts][d_ffn][d_model], down [n_experts][d_model][d_ffn],
 * each with fp16 scales/biases per 64-code group; x fp16 [n][d_model];
 * out [n][d_model]. Experts are visited once per step: the (token, slot)
 * pairs are grouped by expert (kvp_moe_permute's stable order; for
 * n * k <= 512 on the 4/8-bit matrix-core path the gate/up launch builds
 * that order itself) so each expert's weights stream from HBM once however
 * many tokens chose it. A pair naming no expert (idx >= n_experts) adds
 * nothing.
 * n * k <= 8192. workspace: kvp_moe_swiglu_workspace_bytes(n, k, n_experts,
 * d_model, d_ffn). */
size_t kvp_moe_swiglu_workspace_bytes(int n, int k, int n_experts, int d_model, int d_ffn);
int kvp_moe_swiglu(const void* x, const uint32_t* idx, const float* gate,
                   const uint32_t* gate_wq, const void* gate_scales, const void* gate_biases,
                   const uint32_t* up_wq, const void* up_scales, const void* up_biases,
                   const uint32_t* down_wq, const void* down_scales, const void* down_biases,
                   void* out, int out_dtype, int n, int k, int n_experts, int d_model,
                   int d_ffn, int bits, void* workspace, size_t workspace_bytes, void* stream);

/* Kernel-selection overrides, for tiling sweeps and A/B tests only: the
 * library's own choice applies to every key that is not set, and nothing
 * else (no environment variable) changes which kernel a call runs. Keys:
 * "qmv_path" (1 streaming, 2 resident, 3 chunked, 4 matrix cores,
 * 5 persistent), "qmv_per_cu", "qmv_blocks", "qmv_kw", "qmv_rw",
 * "qmv_mfma_tiles", "moe_valu", "moe_kq", "moe_permute", "moe_down_combine".
 * value -1 restores the library's choice. Process-wide; set before the calls it should
 * affect. No counterpart in the reference (its kernels have one body). */
int kvp_set_tuning(const char* key, int value);
int kvp_get_tuning(const char* key, int* value);

/* Routing from logits and the SwiGLU experts in one call: the result of
 * kvp_moe_route_logits (idx, gate written as it writes them) followed by
 * kvp_moe_swiglu, same arguments and workspace. For up to 4 tokens on the
 * 4/8-bit matrix-core path (n * k <= 512, n_experts <= 256) every gate/up
 * block routes the tokens itself, so no routing launch precedes the experts;
 * otherwise the routing kernel runs first. No reference counterpart: the
 * reference's routing and dispatch are separate kernels
 * (kernelverify/pack/moe_dispatch.py:39-138). */
int kvp_moe_route_swiglu(const float* logits, const void* x, uint32_t* idx, float* gate,
                         const uint32_t* gate_wq, const void* gate_scales,
                         const void* gate_biases, const uint32_t* up_wq, const void* up_scales,
                         const void* up_biases, const uint32_t* down_wq, const void* down_scales,
                         const void* down_biases, void* out, int out_dtype, int n, int k,
                         int n_experts, int d_model, int d_ffn, int bits, void* workspace,
                         size_t workspace_bytes, void* stream);

/* HBM roofline probe kernels (replaces bench/metal/roofline_probe.mm:35-144
 * stream_read / stream_copy). `n_bytes` multiple of 16. read_sink receives a
 * per-block value so the loads cannot be removed. */
int kvp_probe_stream_read(const void* src, size_t n_bytes, float* read_sink, int blocks,
                          void* stream);
int kvp_probe_stream_copy(const void* src, void* dst, size_t n_bytes, int blocks,
                          void* stream);

/* Tunable read probe (the sweep behind the measured ceiling). Each block
 * reads whole tiles of threads x unroll 16-byte units, every lane's `unroll`
 * loads issued before any is used; flags bits 0-1 pick the load (0 plain,
 * 1 non-temporal, 2 buffer), bit 2 gives each block one contiguous range of
 * tiles instead of grid-strided tiles. threads in {64, 128, 256, 512, 1024},
 * unroll in {1, 2, 4, 8, 16}; `sink` receives one float per block. */
int kvp_probe_read_tiled(const void* src, size_t n_bytes, float* sink, int blocks, int threads,
                         int unroll, int flags, void* stream);

/* Compute-ceiling probes (replaces bench/metal/roofline_probe.mm:103-144, the
 * fp32 / fp16 FMA peaks): kind 0 fp32 FMA, 1 V_DOT2_F32_F16, 2
 * V_MFMA_F32_16X16X32_F16, in 256-thread blocks of independent chains.
 * kvp_probe_compute_flops gives the flops one launch performs. */
double kvp_probe_compute_flops(int kind, int blocks, int iters);
int kvp_probe_compute(int kind, int blocks, int iters, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVPACK_H_ */
