/*
 * gdn2_hip.h -- C ABI of the MI355X (gfx950) GDN-2 attention library
 * (libgdn2_hip.so, built from gdt2_tilelang_amd/csrc).
 *
 * Plain pointers and sizes only. Every tensor is device memory owned by the
 * caller; the library never allocates or frees. Sequence tensors are
 * [B, s_alloc, H, D] contiguous with D fastest and a call works on tokens
 * [t0, t0 + n) of that allocation; g is fp32 natural-log decay (<= 0); the
 * state is fp32 [B, H, DK, DV] contiguous. Grouped heads: the key-side tensors
 * q, k, b, g may have HK heads with HK dividing the H heads of v, w, o and the
 * state; value head h then reads key head h / (H / HK) (HK = H: no grouping;
 * the reference repeats the key heads instead, gdn2/attention.py:295-297).
 * Work is enqueued on `stream`
 * (a hipStream_t; NULL = the default stream) with no host synchronisation.
 *
 * Return value: 0 on success, a negative GDN2_ERR_* for a rejected argument
 * (nothing was launched), or a positive hipError_t from the launch.
 *
 * The reference (amaranthine09/GDT2_TileLang) has no C ABI: its kernels are
 * TileLang JIT objects called from Python. Each entry point below names the
 * reference call site it replaces.
 */
#ifndef GDN2_HIP_H
#define GDN2_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes for q, k, v, b, w and for the output o */
#define GDN2_DTYPE_F32 0
#define GDN2_DTYPE_BF16 1
#define GDN2_DTYPE_F16 2

#define GDN2_ERR_ARG (-1)    /* null pointer, negative size, bad dtype code */
#define GDN2_ERR_SHAPE (-2)  /* head dim / token count the kernels do not support */
#define GDN2_ERR_SCRATCH (-3) /* call needs more than the no-alloc entry point's fixed scratch */

/* Library ABI version (bumped on any signature or layout change). */
int gdn2_hip_version(void);

/* Static description of a status code. */
const char* gdn2_hip_status_string(int status);

/*
 * Decode n tokens with the state resident on chip: per token
 *   S <- diag(exp g) S ; u = w*v - S^T (b*k) ; S <- S + k u^T ; o = scale S^T q
 * state is updated in place; o is [B, s_alloc, H, DV] in out_dtype.
 * Supports DK in {32, 64, 128, 256}, DV a multiple of 32, any n >= 0.
 * Replaces: decode_multi_kernel(...)(...) in gdn2/inference.py:347-353
 * (gdn2_decode) and decode_step_kernel(...)(...) in gdn2/inference.py:190-196
 * (gdn2_decode_step, which is n = 1 with s_alloc = 1).
 */
int gdn2_hip_decode(const void* q, const void* k, const void* v, const float* g, const void* b,
                    const void* w, int in_dtype, float* state, void* o, int out_dtype, int B,
                    int H, int HK, int DK, int DV, long s_alloc, long t0, long n, float scale,
                    void* stream);

/* Bytes of workspace gdn2_hip_chunk_local / gdn2_hip_prefill_chunks need for
 * n_tokens tokens (rounded up to whole 64-token chunks) of B x HK key heads; 0 for an unsupported
 * DK. One record per key head and chunk (58 112 B at DK = 128, 41 472 B at DK = 64). The records
 * depend on q, k, b, g only, so grouped value heads share them. */
size_t gdn2_hip_prefill_workspace_bytes(int B, int HK, int DK, long n_tokens);

/*
 * Prefill stage 1 (chunk-local, fully parallel): for every 64-token chunk of
 * tokens [t0, t0 + n_tokens) build the log2-space decay cumsum, the Aqk / Akk
 * blocks, Ai = (I + Akk)^-1 and the WY factors, and write one record per chunk
 * into `workspace`. q, k, b, g are [B, s_alloc, HK, DK] (HK key heads; pass
 * the head count of those tensors). DK in {64, 128}. n_tokens need not be a
 * multiple of 64: the last chunk's rows past n_tokens are read as zeros (they
 * are never loaded), which leaves the state and the other outputs unchanged.
 * Replaces: wy_stages kernels 1-5 in gdn2/forward.py:801-826
 * (cumsum, intra_diag, inter_blocks, solve, wy).
 */
int gdn2_hip_chunk_local(const void* q, const void* k, const void* b, const float* g,
                         int in_dtype, void* workspace, int B, int HK, int DK, long s_alloc,
                         long t0, long n_tokens, float scale, void* stream);

/*
 * Prefill stage 2 (sequential over chunks, parallel over B*H*DV-tiles): the
 * state scan fused with the output; reads the stage-1 records and v, w.
 * state_in may be NULL (zero state) and may equal state_out. DV a multiple of 16.
 * v, w, o and the state have H value heads; value head h reads the records of
 * key head h / (H / HK).
 * Replaces: prefill_scan_kernel(...)(...) in gdn2/inference.py:544-550 and the
 * state_kernel + output_kernel pair in gdn2/forward.py:879-892.
 */
int gdn2_hip_prefill_scan(const void* v, const void* w, int in_dtype, const void* workspace,
                          const float* state_in, float* state_out, void* o, int out_dtype, int B,
                          int H, int HK, int DK, int DV, long s_alloc, long t0, long n_tokens,
                          void* stream);

/*
 * Both prefill stages back to back on one stream: o[t0 : t0+n_tokens] and the
 * state after the last token (n_tokens any count >= 1; o rows past it are not
 * written). Replaces the device branch of gdn2_prefill
 * (gdn2/inference.py:542-550) and of chunk_gdn2_fwd (gdn2/forward.py:870-895).
 */
int gdn2_hip_prefill_chunks(const void* q, const void* k, const void* v, const float* g,
                            const void* b, const void* w, int in_dtype, const float* state_in,
                            float* state_out, void* o, int out_dtype, void* workspace, int B,
                            int H, int HK, int DK, int DV, long s_alloc, long t0, long n_tokens,
                            float scale, void* stream);

/*
 * gdn2_hip_prefill_chunks without the workspace argument: the chunk records go
 * to a scratch array the library holds in device memory, one per GPU, of
 * GDN2_NOALLOC_SCRATCH_BYTES (64 MiB of gdn2_hip_prefill_workspace_bytes: e.g.
 * 2304 tokens of 32 key heads, 9216 tokens of 8 key heads).
 * A larger call returns GDN2_ERR_SCRATCH and launches nothing (prefill it in
 * segments, passing state_out back as state_in). The call allocates nothing:
 * no hipMalloc / hipFree, nothing from a caching allocator, so it can run
 * where allocation is not allowed. Every call on one GPU shares that GPU's
 * scratch, so calls that overlap in time on one GPU (different streams, or
 * different threads) race: serialise them. Results equal
 * gdn2_hip_prefill_chunks on the same arguments.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (HIP graph capture, serving loops, harnesses that forbid it).
 */
#define GDN2_NOALLOC_SCRATCH_BYTES (64L * 1024 * 1024)
int gdn2_hip_prefill_chunks_noalloc(const void* q, const void* k, const void* v, const float* g,
                                    const void* b, const void* w, int in_dtype, const float* state_in,
                                    float* state_out, void* o, int out_dtype, int B, int H, int HK, int DK,
                                    int DV, long s_alloc, long t0, long n_tokens, float scale, void* stream);

/*
 * Both prefill stages over a packed variable-length batch: nseq sequences
 * concatenated in one [T, H, D] allocation (q, k, b, g with HK heads; v, w, o
 * with H), sequence i holding tokens [cu_seqlens[i], cu_seqlens[i+1]) and
 * running its own recurrence from state_in[i] (state_in NULL: zeros) to
 * state_out[i] (both fp32 [nseq, H, DK, DV]; they may be equal). cu_seqlens is
 * int32 in device memory, nseq + 1 entries, 0 = cu[0] <= cu[1] <= ... <= cu[nseq]
 * = T (empty sequences allowed: their state is copied through). The library
 * cannot check the offsets without a host sync; it clamps them into [0, T],
 * so malformed offsets give wrong results but no access outside the buffers.
 * One chunk-local launch covers every sequence's chunks, one scan launch every
 * (sequence, value head, tile). DK in {64, 128}; DV a multiple of 16.
 * Workspace: gdn2_hip_prefill_varlen_workspace_bytes (ceil(T/64) + nseq
 * record slots per key head).
 * Replaces: gdn2_attention(..., cu_seqlens=...) (gdn2/attention.py:142-145),
 * which the reference rejects with NotImplementedError.
 */
size_t gdn2_hip_prefill_varlen_workspace_bytes(int nseq, int HK, int DK, long T);
int gdn2_hip_prefill_varlen(const void* q, const void* k, const void* v, const float* g,
                            const void* b, const void* w, int in_dtype, const int* cu_seqlens, int nseq,
                            const float* state_in, float* state_out, void* o, int out_dtype,
                            void* workspace, int H, int HK, int DK, int DV, long T, float scale,
                            void* stream);

/*
 * GatedDeltaNet2 layer prologue (one launch per prefill segment or decode
 * block): for the B x S tokens of the raw projections xq, xk [.., HK*DK],
 * xv, xw [.., H*DV], xb, xf [.., HK*DK] (row strides ld_* in elements, all in
 * act_dtype), compute
 *   q, k = L2-normalised (per DK-channel head) SiLU(causal depthwise conv(x))
 *   v    = SiLU(causal depthwise conv(xv))
 *   b    = sigmoid(xb) * erase_scale,  w = sigmoid(xw)
 *   g    = -exp(a_log[hk]) * softplus(xf + dt_bias[hk, :])        (fp32)
 * into contiguous q, k, b [B, S, HK, DK], v, w [B, S, H, DV] (act_dtype) and
 * g [B, S, HK, DK] (fp32). The conv (width conv_k <= 4, weights conv_w
 * [C, conv_k] and bias conv_b [C] in act_dtype, C = 2*HK*DK + H*DV, channel
 * order q | k | v) continues from conv_in [B, C, conv_k - 1] (NULL: zeros) and
 * writes the last conv_k - 1 conv inputs to conv_out (same layout, distinct
 * buffer; NULL: not written). conv_w NULL: no conv (and no SiLU).
 * DK/8 must be a power of two <= 64 and DV a multiple of 8; the row strides
 * multiples of 8 and every x / output / conv pointer 16-byte aligned.
 * Replaces: the layer's q/k/v conv, F.normalize and gate/decay ops in
 * gdn2/attention.py (_ShortConv.decode :206-215, _gates :290-293, the
 * normalisation in prefill/decode :360-402).
 */
int gdn2_hip_layer_prologue(const void* xq, const void* xk, const void* xv, const void* xb,
                            const void* xw, const void* xf, long ld_q, long ld_k, long ld_v,
                            long ld_b, long ld_w, long ld_f, int act_dtype, const void* conv_w,
                            const void* conv_b, int conv_k, const void* conv_in, void* conv_out,
                            const float* a_log, const float* dt_bias, float erase_scale, void* q,
                            void* k, void* v, void* b, void* w, float* g, int B, long S, int H,
                            int HK, int DK, int DV, void* stream);

/*
 * The layer prologue over a packed variable-length batch: T tokens of nseq
 * sequences in one row (cu_seqlens as for gdn2_hip_prefill_varlen, int32 in
 * device memory). Each token's conv window starts at its own sequence's first
 * token; the rows before it come from that sequence's cached conv tail,
 * conv_in [nseq, C, conv_k - 1] (NULL: zeros, a fresh sequence). conv_out
 * [nseq, C, conv_k - 1] (NULL: not written; distinct from conv_in) receives
 * every sequence's new tail, the last conv_k - 1 conv inputs, earlier entries
 * coming from its old tail (an empty sequence keeps its tail). The L2 norms,
 * gates and decay are per token as in gdn2_hip_layer_prologue.
 * Replaces: the same ops as gdn2_hip_layer_prologue for
 * GatedDeltaNet2.forward(..., cu_seqlens=...) (gdn2/attention.py:299-358), whose
 * cu_seqlens the reference's op rejects.
 */
int gdn2_hip_layer_prologue_varlen(const void* xq, const void* xk, const void* xv, const void* xb,
                                   const void* xw, const void* xf, long ld_q, long ld_k, long ld_v,
                                   long ld_b, long ld_w, long ld_f, int act_dtype, const void* conv_w,
                                   const void* conv_b, int conv_k, const void* conv_in, void* conv_out,
                                   const float* a_log, const float* dt_bias, float erase_scale, void* q, void* k,
                                   void* v, void* b, void* w, float* g, const int* cu_seqlens, int nseq, long T,
                                   int H, int HK, int DK, int DV, void* stream);

/*
 * Few-row linear layer y = x W^T: x [M, K] (row stride ldx), W [N, K] (the
 * nn.Linear weight, contiguous), y [M, N] (row stride ldy), all in dtype, fp32
 * accumulation. M <= 8, K and ldx multiples of 8, x and W 16-byte aligned.
 * Bound by reading W once; for decode steps of a few tokens it replaces the
 * layer's projection GEMMs (gdn2/attention.py:440-454 and o_proj :268, :414,
 * which torch runs through hipBLASLt).
 */
int gdn2_hip_gemv(const void* x, long ldx, const void* W, void* y, long ldy, int dtype, int M, int N,
                  int K, void* stream);

/*
 * Training backward of the attention op: given the forward inputs and the
 * gradient d_out [B, S, H, DV] (do_dtype) of o, and optionally the gradient
 * d_final_state [B, H, DK, DV] fp32 of the final state, writes
 *   dq, dk, db [B, S, HK, DK] and dv, dw [B, S, H, DV] in in_dtype,
 *   dg [B, S, HK, DK] fp32, and, if d_initial_state is not null, the
 *   gradient of initial_state (fp32 [B, H, DK, DV]; null initial_state means
 *   zeros) into d_initial_state.
 * Chunkwise form in fp32 (chunk 64): per-chunk local factors, a forward scan
 * of the chunk-entry states, a reverse scan of the state gradients, per-chunk
 * gradients, and the sum over the value heads of each key head. DK in {32,
 * 64, 128}, DV a multiple of 16 (<= 4096). `workspace` (256-byte aligned)
 * holds gdn2_hip_backward_workspace_bytes(B, H, HK, DK, DV, S) bytes, which
 * grows linearly in B * S: with NC = ceil(S / 64) it is the fp32 chunk
 * records (B * HK * NC * 65.6 K floats at DK = 128), two fp32 per-chunk state
 * checkpoints (2 * B * H * NC * DK * DV * 4), with grouped heads (H > HK)
 * four fp32 per-value-head partial gradients (4 * B * S * H * DK * 4), the
 * per-chunk gradient sums, and room for an fp32 copy of d_out (used when
 * do_dtype is neither in_dtype nor fp32). Examples at DK = DV = 128: B=2
 * S=4096 H=HK=16: 1.14 GB; B=1 S=32768 H=HK=16: 4.6 GB.
 * Replaces: chunk_gdn2_bwd (gdn2/backward.py:912-994), called from
 * _GDN2Function.backward (gdn2/attention.py:79-99).
 */
size_t gdn2_hip_backward_workspace_bytes(int B, int H, int HK, int DK, int DV, long S);
int gdn2_hip_backward(const void* q, const void* k, const void* v, const float* g, const void* b, const void* w,
                      int in_dtype, float scale, const float* initial_state, const void* d_out, int do_dtype,
                      const float* d_final_state, void* dq, void* dk, void* dv, float* dg, void* db, void* dw,
                      float* d_initial_state, void* workspace, int B, long S, int H, int HK, int DK, int DV,
                      void* stream);

/*
 * Training backward of packed variable-length sequences (the backward of
 * gdn2_hip_prefill_varlen's forward): one row of T tokens holding nseq
 * sequences, sequence s at tokens [cu_seqlens[s], cu_seqlens[s+1]) (int32,
 * device memory, non-decreasing from 0 to T), each its own recurrence from
 * initial_state[s]. Tensors as for gdn2_hip_backward with B = 1 and S = T;
 * initial_state, d_final_state and d_initial_state are [nseq, H, DK, DV]. An
 * empty sequence passes its final-state gradient through to d_initial_state.
 * All sequences run in one set of launches: the per-chunk kernels take the
 * forward's record slots (chunk c of sequence s at slot s + floor(cu[s]/64)
 * + c; slots between sequences exit at once) and the scans run per
 * (sequence, value head, 16 columns). Workspace (256-byte aligned):
 * gdn2_hip_backward_varlen_workspace_bytes, the dense formula with
 * ceil(T/64) + nseq chunk slots per head.
 * No reference counterpart: the reference raises for cu_seqlens
 * (gdn2/attention.py:142-145); this replaces one gdn2_hip_backward call per
 * sequence.
 */
size_t gdn2_hip_backward_varlen_workspace_bytes(int nseq, int H, int HK, int DK, int DV, long T);
int gdn2_hip_backward_varlen(const void* q, const void* k, const void* v, const float* g, const void* b,
                             const void* w, int in_dtype, float scale, const float* initial_state,
                             const void* d_out, int do_dtype, const float* d_final_state, void* dq, void* dk,
                             void* dv, float* dg, void* db, void* dw, float* d_initial_state, void* workspace,
                             const int* cu_seqlens, int nseq, long T, int H, int HK, int DK, int DV,
                             void* stream);

/*
 * One GatedDeltaNet2 decode call of n tokens for B sequences (B*n <= 8), as
 * three launches on one stream: the projections (the fused weight w_proj
 * [4*HK*DK + 3*H*DV, hidden], rows q | k | v | b | w | f | o_gate) with the
 * layer prologue applied to their sums (conv with conv_in -> conv_out, SiLU,
 * gates, decay), the recurrence on `state` (fp32 [B, H, DK, DV], updated in
 * place) with the q / k L2 norm, and o_proj (w_out [hidden, H*DV]) with the
 * gated RMSNorm (norm_w fp32 [DV]) applied to its input. The result agrees,
 * to the rounding of the activation dtype, with
 * gdn2_hip_gemv + gdn2_hip_layer_prologue + gdn2_hip_decode +
 * gdn2_hip_layer_epilogue + gdn2_hip_gemv run stage by stage.
 * x [B*n, hidden] and out [B*n, hidden] in dtype. Intermediates live in
 * `workspace` (256-byte aligned, gdn2_hip_layer_decode_workspace_bytes).
 * Replaces: GatedDeltaNet2.decode / step (gdn2/attention.py:417-478).
 */
size_t gdn2_hip_layer_decode_workspace_bytes(int B, int n, int H, int HK, int DK, int DV, int dtype);
int gdn2_hip_layer_decode(const void* x, const void* w_proj, const void* conv_w, const void* conv_b,
                          int conv_k, const void* conv_in, void* conv_out, const float* a_log,
                          const float* dt_bias, float erase_scale, float* state, const float* norm_w,
                          float norm_eps, const void* w_out, void* out, void* workspace, int dtype, int B,
                          int n, int hidden, int H, int HK, int DK, int DV, float scale, void* stream);

/*
 * GatedDeltaNet2 layer epilogue: per token and value head,
 *   out = o * rsqrt(mean(o^2) + eps) * weight * silu(gate)
 * o [B, S, H, DV] contiguous in o_dtype; gate and out rows of H*DV in
 * out_dtype with row strides ld_gate / ld_out; weight [DV] fp32.
 * Replaces: _GatedRMSNorm.forward (gdn2/attention.py:218-229).
 */
int gdn2_hip_layer_epilogue(const void* o, int o_dtype, const void* gate, long ld_gate,
                            const float* weight, float eps, void* out, int out_dtype, long ld_out,
                            int B, long S, int H, int DV, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_HIP_H */
