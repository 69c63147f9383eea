/*
 * mx_kernels.h — C-ABI of the MI355X (gfx950) quant-inference kernel path.
 *
 * One shared library (libmxkernels.so) exports these entry points.  Every
 * pointer argument is a device pointer the caller allocated (for instance a
 * torch tensor's data_ptr()); every call is asynchronous on the HIP stream
 * passed as `stream` (NULL = the legacy default stream) and returns an int
 * status: MX_OK (0) or a negative MX_ERR_* code.  No entry point exits,
 * aborts, synchronises the device or allocates device memory.  Arguments
 * are validated before anything is launched — for an entry point that
 * launches several kernels, the arguments of all of them — so any error
 * return other than MX_ERR_LAUNCH means nothing was enqueued.
 * MX_ERR_LAUNCH reports that the HIP runtime refused a launch; in a
 * multi-kernel entry point the kernels before it may already be enqueued.
 * The library holds no per-call state: calls are re-entrant and may be
 * issued from several host threads on different streams.
 *
 * The reference (baladithyab/cuda-oxide-bench) launches each of these
 * operations from a Python harness through `ct.launch(stream.ptr, grid,
 * kernel, (arrays...))` on caller-allocated, row-major, contiguous device
 * arrays; the citation on each declaration names the launch it replaces.
 */
#ifndef MX_KERNELS_H
#define MX_KERNELS_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define MX_OK 0
#define MX_ERR_NULL (-1)        /* a required pointer is NULL                    */
#define MX_ERR_SHAPE (-2)       /* a size is <= 0, inconsistent or too large     */
#define MX_ERR_ALIGN (-3)       /* pointer / leading dimension not 16-B aligned  */
#define MX_ERR_DTYPE (-4)       /* unsupported element-type code                 */
#define MX_ERR_WORKSPACE (-5)   /* workspace missing or smaller than required    */
#define MX_ERR_ALIAS (-6)       /* an output overlaps an input it may not alias  */
#define MX_ERR_LAUNCH (-7)      /* the HIP runtime rejected the kernel launch    */
#define MX_ERR_UNSUPPORTED (-8) /* valid request this build has no kernel for    */

/* ---- element-type codes for the 16-bit I/O tensors --------------------- */
#define MX_DTYPE_BF16 0
#define MX_DTYPE_F16 1

/* Human-readable name of a status code (static storage, never NULL). */
const char* mx_strerror(int code);

/* Library version string, e.g. "mxkernels 0.1.0 gfx950". */
const char* mx_version(void);

/*
 * bf16 GEMM:  C[M,N] = A[M,K] · B[K,N]
 * A, B, C row-major bf16 with leading dimensions lda >= K, ldb >= N,
 * ldc >= N (in elements).  fp32 accumulation, C rounded to bf16 (RNE).
 * Requires K % 8 == 0, N % 8 == 0, lda/ldb/ldc % 8 == 0 and 16-byte aligned
 * pointers; M, N, K otherwise arbitrary (ragged edges are zero-padded).
 * Shapes that run the register-staged kernel (K % 32 != 0, or small grids)
 * take lda < 2^30 / BM (BM = 256, 128 or 64 rows per tile, so at least 4M
 * elements) and ldb < 16M elements; larger strides return MX_ERR_SHAPE.
 * Replaces: cutile-matmul-tc-bf16/main.py:117-118 (ct.launch of the
 * `matmul_bf16` kernel defined at :59-78) and the bf16 row of
 * cutile-matmul-tiled-mixed/main.py:121-130.
 */
int mx_gemm_bf16(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb,
                 int ldc, void* stream);

/*
 * Strided-batched bf16 GEMM:  for i < batch,
 *   C_i[M,N] = A_i[M,K] · B_i[K,N],  X_i = X + i * strideX (elements)
 * with the layout and requirements of mx_gemm_bf16 per item, batch <= 65535,
 * strides >= 0 and multiples of 8.  Items may be interleaved views, e.g.
 * head h of a [B, H, d] activation (A + h*d, lda = H*d).  This path uses it
 * for the per-head MLA weight products either side of the latent decode:
 * q_lat = q_nope · W_UK[h] and o = o_lat · W_UV[h].
 * Replaces: the per-head up-projections of the absorbed MLA decode that
 * analysis/wave15-attention-research/MECHANISMS.md:91-94, 115-120 describes
 * (the reference has no kernel for them).
 */
int mx_gemm_bf16_batched(const void* A, const void* B, void* C, int batch, int M, int N, int K,
                         int lda, int ldb, int ldc, long long strideA, long long strideB,
                         long long strideC, void* stream);

/*
 * fp8 block-scaled GEMM:
 *   C[m,n] = sum_kb sA[m,kb] * sB[kb,n/128] * sum_{k in block kb} A[m,k] * B[k,n]
 * A[M,K], B[K,N] row-major OCP e4m3 ("e4m3fn", torch.float8_e4m3fn) bytes;
 * sA[M, K/128] and sB[K/128, ceil(N/128)] row-major fp32 dequantisation
 * scales (1x128 blocks of A, 128x128 blocks of B); C[M,N] row-major bf16.
 * fp32 accumulation with the scale applied once per 128-deep K block.
 * Requires K % 128 == 0, N % 16 == 0, 16-byte aligned A, B, C.
 * Replaces: mojo-matmul-fp8/matmul_fp8.mojo:48-218 (matmul_fp8_kernel,
 * e4m3 x e4m3 -> f32, launched at :285-289), extended with the block
 * scaling and bf16 output this path specifies.
 */
int mx_gemm_fp8_bs(const void* A, const float* sA, const void* B, const float* sB, void* C, int M,
                   int N, int K, void* stream);

/*
 * fp8 activation quantisation (the producer of mx_gemm_fp8_bs's A operand):
 * for every row m and 128-wide column block kb of X[M,K] (bf16 or f16,
 * leading dimension ldx >= K, in elements):
 *   scales[m,kb] = max_{k in kb} |X[m,k]| / 448   (1.0 for an all-zero block)
 *   Q[m,k]       = e4m3fn(RNE(clamp(X[m,k] / scales[m,kb], -448, 448)))
 * Q is [M,K] row-major bytes, scales [M, K/128] fp32.  Non-finite values
 * follow the same recipe: a block holding a NaN has scale 1 (its amax is
 * NaN, not > 0), a block with an infinite amax has scale +inf (its finite
 * values encode to +-0, its infinities to NaN), and NaN encodes to a NaN
 * code (0x7F or 0xFF).  Requires K % 128 == 0,
 * ldx % 8 == 0, 16-byte aligned X and Q.
 * Replaces: the host-side generation of the fp8 GEMM operands
 * (mojo-matmul-fp8/matmul_fp8.mojo:262-270 fills them on the CPU), extended
 * with the 1x128 block scaling this path specifies.
 */
int mx_quant_fp8_act(const void* X, void* Q, float* scales, int M, int K, int ldx, int dtype,
                     void* stream);

/*
 * Fused grouped-query attention forward (flash-attention style, one pass):
 *   O[b,h,s,:] = softmax_t( scale * Q[b,h,s,:]·K[b,h/G,t,:] + mask ) · V[b,h/G,t,:]
 * with G = Hq / Hkv and mask = -inf for t > s when causal != 0.
 * Q, O: [B, Hq, S, D]; K, V: [B, Hkv, S, D]; contiguous, dtype as given
 * (MX_DTYPE_BF16 or MX_DTYPE_F16).  fp32 scores, online softmax and
 * accumulation; O rounded to the I/O dtype.  D must be 64 or 128,
 * Hq % Hkv == 0; S arbitrary (>= 1).
 * Replaces: cutile-attn-gqa/main.py:249-252 (ct.launch of `gqa_fwd`,
 * kernel at :64-170, non-causal f16) — the causal flag and bf16 are the
 * extensions this path specifies.
 */
int mx_gqa_fwd(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S,
               int D, float scale, int causal, int dtype, void* stream);

/*
 * mx_gqa_fwd with an explicit tile: block_m query rows of each head per
 * workgroup, block_n keys per LDS stage, wave_m query rows per wave.
 * block_n must be 64 (the kernels' key stage).  A workgroup covers hpw =
 * waves * wave_m / block_m heads of one KV group, a whole number dividing
 * both the wave count and G = Hq / Hkv.  wave_m = 32 runs 8 waves (two per
 * SIMD) when that allows, else 4 waves (two workgroups per CU); wave_m = 64
 * runs 4 waves (one per SIMD, 512 registers; each K/V fragment feeds two
 * MFMAs).  A tile no kernel has returns MX_ERR_UNSUPPORTED before anything
 * is enqueued.  Any S is
 * accepted (ragged query and key tiles are masked).  mx_gqa_fwd runs
 * block_m = mx_gqa_fwd_default_block_m(Hq, Hkv, D), block_n 64, wave_m 32.
 * Replaces: cutile-attn-gqa/main.py:202-230 (pick_blocks with the
 * --block-m / --block-n overrides, each pair compiled by make_gqa_kernel,
 * :64-66) and the launch at :249-252.
 */
int mx_gqa_fwd_tile(const void* Q, const void* K, const void* V, void* O, int B, int Hq, int Hkv, int S,
                    int D, float scale, int causal, int dtype, int block_m, int block_n, int wave_m,
                    void* stream);

/* MX_OK if mx_gqa_fwd_tile has a kernel for this tile at (Hq, Hkv, D), else
 * MX_ERR_UNSUPPORTED (MX_ERR_SHAPE for invalid head counts or D).  Host
 * logic only: no GPU call. */
int mx_gqa_fwd_tile_check(int Hq, int Hkv, int D, int block_m, int block_n, int wave_m);

/* BLOCK_M of mx_gqa_fwd's default tile (8 waves of 32 queries over hpw =
 * 4, 2 or 1 heads of a KV group as G allows: 256 / hpw), or MX_ERR_SHAPE.
 * Host logic only. */
int mx_gqa_fwd_default_block_m(int Hq, int Hkv, int D);

/* Registers per lane (numRegs) and scratch bytes per lane (spills) of the
 * gfx950 kernel that mx_gqa_fwd_tile runs for this tile; what the
 * reference's block sweep reads from its compiled kernels
 * (cutile-attn-gqa/sweep_block_m.py, lmem_check).  Needs the HIP runtime. */
int mx_gqa_fwd_tile_info(int Hq, int Hkv, int D, int dtype, int causal, int block_m, int block_n, int wave_m,
                         int* vgprs, int* scratch_bytes);

/*
 * Pre-projected MLA prefill attention (multi-head, every head its own K/V):
 *   O[b,h,s,:] = softmax_t( scale * Q[b,h,s,:]·K[b,h,t,:] + mask ) · V[b,h,t,:]
 * Q, K: [B, H, S, d_qk]; V, O: [B, H, S, d_v]; contiguous bf16 or f16;
 * mask = -inf for t > s when causal != 0.  (d_qk, d_v) must be (192, 128)
 * (DeepSeek-V3: 128 nope + 64 rope, v 128), (96, 64), (128, 128) or
 * (64, 64); the qk head dim is used as is, not padded.  Same kernel family
 * as mx_gqa_fwd (one KV head per query head).
 * Replaces: cutile-attn-mla/main.py:250-253 (ct.launch of `mla_fwd`,
 * kernel at :81-163, which zero-pads qk_head_dim 192 to 256 on the host,
 * :179-206); causal and bf16 are the extensions this path specifies.
 */
int mx_mla_prefill_fwd(const void* Q, const void* K, const void* V, void* O, int B, int H, int S, int d_qk,
                       int d_v, float scale, int causal, int dtype, void* stream);

/*
 * MLA absorbed decode (one query token per sequence, latent KV cache):
 *   O[b,h,:] = softmax_t( scale * Q[b,h,:]·KV[b,t,:] ) · KV[b,t,0:d_latent]
 * Q[B,H,d_latent+d_rope], KV[B,T,d_latent+d_rope], O[B,H,d_latent], all
 * contiguous bf16.  d_latent = 512 and d_rope = 64 are supported (the
 * DeepSeek-V3 latent width 576).  The kernel splits T across workgroups
 * and merges the partial softmax states; the caller passes a device
 * workspace of at least mx_mla_decode_workspace(B, H, T, d_latent) bytes.
 * Replaces: cutile-attn-mla/main.py:250-253 (ct.launch of `mla_fwd`,
 * kernel at :81-163).  The reference kernel attends over pre-projected
 * per-head K/V; this entry point is the weight-absorbed latent form of the
 * same softmax attention (analysis/wave15-attention-research/MECHANISMS.md:91-94).
 */
int mx_mla_decode(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent,
                  int d_rope, float scale, void* workspace, size_t ws_bytes, void* stream);

/* Bytes of device workspace mx_mla_decode needs for this problem (0 on
 * invalid sizes). */
size_t mx_mla_decode_workspace(int B, int H, int T, int d_latent);

/* Number of slices T is split into (one workgroup per sequence, slice and
 * 128-head group; 1 = no merge pass) for this problem, 0 on invalid sizes.
 * No counterpart in the reference (its kernel does not split T); harnesses
 * report it next to the timing. */
int mx_mla_decode_splits(int B, int H, int T);

/*
 * Allocation-free MLA decode: mx_mla_decode without a workspace argument.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The same kernels and results as mx_mla_decode; the split
 * partials go to a library-owned device array of MX_MLA_SCRATCH_BYTES per
 * GPU.  The array sits in a code object of its own (csrc/mla_noalloc.hip),
 * so only processes that use this entry point hold it: with the HIP
 * runtime's deferred code-object loading, a GPU holds it from the first
 * call of this entry point there until the process ends.  Problems
 * whose mx_mla_decode_workspace(B, H, T, d_latent) exceeds that size return
 * MX_ERR_WORKSPACE.  All calls on one GPU share its array: calls that
 * overlap on one GPU (concurrent streams or host threads) race and must be
 * serialised by the caller.  The caller still allocates Q, KV and O.
 */
#define MX_MLA_SCRATCH_BYTES (128u << 20)
int mx_mla_decode_noalloc(const void* Q, const void* KV, void* O, int B, int H, int T, int d_latent,
                          int d_rope, float scale, void* stream);

/*
 * The whole weight-absorbed MLA decode step (DeepSeek-V3 form):
 *   q_lat[b,h,:] = q_nope[b,h,:] · W_UK[h]              (d_nope -> 512)
 *   o_lat[b,h,:] = mx_mla_decode with Q = [q_lat, q_rope] over KV[b]
 *   O[b,h,:]     = o_lat[b,h,:] · W_UV[h]                (512 -> d_v)
 * q_nope [B,H,d_nope], q_rope [B,H,64], KV [B,T,576], W_UK [H,d_nope,512],
 * W_UV [H,512,d_v], O [B,H,d_v], all bf16 row-major; fp32 accumulation,
 * q_lat and o_lat rounded to bf16.  The workspace (q_lat, o_lat and the
 * decode's split partials) is sized by mx_mla_decode_absorbed_workspace and
 * must be 256-byte aligned.  d_nope, d_v multiples of 8 (<= 4096).
 * Replaces: the per-head up-projections either side of the absorbed decode
 * that analysis/wave15-attention-research/MECHANISMS.md:77-94, 115-120
 * describes (the reference ships only the pre-projected prefill cell,
 * cutile-attn-mla/main.py:81-163).
 */
int mx_mla_decode_absorbed(const void* q_nope, const void* q_rope, const void* KV, const void* w_uk,
                           const void* w_uv, void* O, int B, int H, int T, int d_nope, int d_v,
                           float scale, void* workspace, size_t ws_bytes, void* stream);
size_t mx_mla_decode_absorbed_workspace(int B, int H, int T);

/*
 * Gated-DeltaNet single-token recurrent decode, per (b, value head hv),
 * with key head hk = hv / (Hv / Hk):
 *   u     = alpha * (k^T S)                  (d_v)
 *   S_out = alpha * S + beta * k (v - u)^T   (d_k x d_v, fp32)
 *   o     = S_out^T q                        (d_v)
 * q, k: [B, Hk, dk]; v, o: [B, Hv, dv] (dtype as given); alpha, beta:
 * [B, Hv] fp32; S_in, S_out: [B, Hv, dk, dv] fp32 with dv contiguous.
 * S_out may equal S_in (in-place update); partial overlap is rejected.
 * dk and dv must be 64, 128, 256 or 512; Hv % Hk == 0.
 * Replaces: cutile-attn-gdn/main.py:268-272 (ct.launch of `gdn_decode`,
 * kernel at :92-185), extended with Hk != Hv grouping.
 */
int mx_gdn_decode(const void* q, const void* k, const void* v, const float* alpha,
                  const float* beta, const float* S_in, float* S_out, void* o, int B, int Hk,
                  int Hv, int dk, int dv, int dtype, void* stream);

/*
 * Width of the d_v column blocks mx_gdn_decode and mx_kda_decode split
 * each head into (one workgroup per (b, head, block)); 0 for unsupported
 * sizes.  For harnesses that report the block (the reference's results.csv
 * `block_v` column and its sweep's `n_blocks`).
 * Replaces: cutile-attn-gdn/main.py:228-246 (`pick_block_v`).
 */
int mx_gdn_decode_block_v(int B, int Hv, int dk, int dv);

/*
 * Kimi-Delta-Attention (KDA) single-token recurrent decode: GDN with a
 * per-channel gate.  Per (b, head h), with e = exp(g[b,h,:]) (d_k values):
 *   S_dec = Diag(e) S
 *   u     = k^T S_dec                        (d_v)
 *   S_out = S_dec + beta * k (v - u)^T       (d_k x d_v, fp32)
 *   o     = S_out^T q                        (d_v)
 * q, k, g: [B, H, dk]; v, o: [B, H, dv]; beta: [B, H] — all in the 16-bit
 * type `dtype` (the reference's f16 gate and beta); S_in, S_out:
 * [B, H, dk, dv] fp32 with dv contiguous.  q is used as given (no 1/sqrt(dk)
 * inside).  S_out may equal S_in; partial overlap is rejected.  dk and dv
 * must be 64, 128, 256 or 512.
 * Replaces: cutile-attn-kda/main.py:357-360 (ct.launch of `kda_decode`,
 * kernel at :187-271; bench launches at :428, :438).
 */
int mx_kda_decode(const void* q, const void* k, const void* v, const void* g, const void* beta,
                  const float* S_in, float* S_out, void* o, int B, int H, int dk, int dv,
                  int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MX_KERNELS_H */
