/*
 * kf950 -- C ABI of the MI355X (gfx950) kernels behind the transformer-layer forward.
 *
 * Plain C: raw device pointers, element strides, sizes, flags and a hipStream_t passed as
 * void*. Every entry point returns a status (KF_OK = 0); on failure kf_last_error() holds a
 * message for the calling thread. No entry point allocates device memory, synchronises the
 * host or throws, so each one may be captured into a HIP graph. Launches are asynchronous
 * on `stream`.
 *
 * The Python reference this replaces has no C boundary of its own: its kernels are Triton
 * functions called from Python. Each entry point below names the reference function whose
 * arguments it carries; the Python wrappers in techjam2026_amd/kernels.py keep those
 * functions' signatures and call these through ctypes.
 */
#ifndef KF950_H
#define KF950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KF_ABI_VERSION 4

/* element types. KF_F16X2 / KF_BF16X2 carry an fp32 value as two 16-bit planes,
 * hi = round(x) and lo = round(x - hi) (the operand format of the split MFMA modes); an
 * entry point taking or producing such a tensor takes a second pointer for the lo plane,
 * which has the same strides as the hi plane. */
enum { KF_F32 = 0, KF_F16 = 1, KF_BF16 = 2, KF_U8 = 3, KF_F16X2 = 4, KF_BF16X2 = 5 };

/* MFMA input precision. The *X3 modes split each fp32 operand into hi + lo 16-bit
 * values and accumulate hi*hi + hi*lo + lo*hi in fp32 (fp32-level accuracy on the
 * fp16/bf16 matrix pipe). KF_MMA_F32 uses the fp32 MFMA (v_mfma_f32_16x16x4_f32). */
enum { KF_MMA_F32 = 0, KF_MMA_F16 = 1, KF_MMA_BF16 = 2, KF_MMA_F16X3 = 3, KF_MMA_BF16X3 = 4,
       /* kf_gemm / kf_gemm_qkv only: A as one fp16 plane (KF_F16), W as the hi/lo planes of
          kf_split(KF_MMA_F16X2); two MFMAs per tile (W_hi.A + W_lo.A): the weights keep
          22 bits, the activations 11 (needs K % 32 == 0). */
       KF_MMA_F16X2 = 5 };

/* status codes */
enum { KF_OK = 0, KF_EINVAL = 1, KF_EUNSUPPORTED = 2, KF_ELAUNCH = 3, KF_EDEVICE = 4 };

/* kf_add_mask_ln flags (kernelforge/ops/layernorm.py:40-86 constexprs) */
enum { KF_LN_HAS_Y = 1, KF_LN_HAS_MASK = 2, KF_LN_MASK_OUT = 4, KF_LN_WRITE_S = 8 };

/* kf_gemm epilogue activations */
enum { KF_ACT_NONE = 0, KF_ACT_GELU_ERF = 1 };

/* kf_flash_fwd flags */
enum {
  KF_FLASH_CAUSAL = 1,
  /* Rows at or beyond kv_len[b] (all padding) are written as zeros instead of computed.
     Exact for the layer stack, whose next step zeroes those rows; not for a standalone
     attention call, which must leave it off. */
  KF_FLASH_SKIP_PAD_ROWS = 2,
  /* KF_MMA_F16X3 only: the probabilities enter P.V as one fp16 plane (rounded to nearest)
     instead of hi + lo, so P.V issues V_hi.P + V_lo.P (two MFMAs per tile, not three);
     q.k keeps all three. Probabilities are in [0, 1], where one fp16 rounding is a relative
     2^-11 on each weight -- a precision option for the per-stage budget. Ignored for
     other modes. */
  KF_FLASH_P16 = 4,
  /* KF_MMA_F16 / KF_MMA_BF16 only: q.k is rounded to the mode's 16-bit type, multiplied by
     sm_scale and rounded again before the softmax, as the reference's narrow forward
     evaluates `matmul(q, k^T) * scale` (kernelforge/ops/flash.py:145-157, ROUND_SCORES;
     `Plan.match_score_rounding`, optimized.py:82, 523). Rejected for other modes. */
  KF_FLASH_ROUND_SCORES = 8,
  /* Single-pass modes at head_dim 64 / 128 run a kernel software-pipelined over 32-key
     chunks (the next chunk's q.k MFMAs issued among this chunk's softmax); this flag
     selects the unpipelined schedule instead (same tile, same masks; results agree to
     rounding). Ignored elsewhere. */
  KF_FLASH_NO_PIPE = 16,
  /* Single-pass modes at head_dim 64 run two 32-row query tiles per wavefront (K and V^T
     fragments shared between them); this flag selects the pipelined kernel with one tile
     per wavefront instead, whose results are the same bit for bit. Ignored elsewhere. */
  KF_FLASH_ONE_TILE = 32,
};

/* Version of this interface (KF_ABI_VERSION). */
int kf_abi_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* kf_last_error(void);

/* 1 if `device` is a gfx950 (MI355X-class) GPU, 0 if not, negative on a HIP error.
 * Replaces the architecture probe of kernelforge/hw.py:149-191 for this library. */
int kf_device_ok(int device);

/* Fused residual add + row mask + LayerNorm.
 * Replaces kernelforge/ops/layernorm.py:101-156 (add_mask_layernorm) and the kernel it
 * launches, :40-86:
 *   s = (x + y) * keep          (fp32; y when KF_LN_HAS_Y, keep when KF_LN_HAS_MASK)
 *   h = (s - mean) * rsqrt(var + eps) * w + b   (biased variance)
 *   h *= keep                   (when KF_LN_MASK_OUT)
 * s is written when KF_LN_WRITE_S. x, y, s, h are [M, d] with row strides ldx, ldy, lds,
 * ldh (elements, unit column stride); keep is [M] (KF_U8 / KF_F32 / KF_F16 / KF_BF16);
 * w, b are [d] of wb_dtype. h may also be KF_F16X2 / KF_BF16X2 planes (h_lo = lo plane). */
int kf_add_mask_ln(const void* x, int x_dtype, int64_t ldx,
                   const void* y, int y_dtype, int64_t ldy,
                   const void* keep, int keep_dtype,
                   const void* w, const void* b, int wb_dtype,
                   void* s_out, int s_dtype, int64_t lds,
                   void* h_out, void* h_lo, int h_dtype, int64_t ldh,
                   int64_t M, int64_t d, float eps, int flags, void* stream);

/* Weight preparation for kf_gemm: hi[i] = round(src[i]) and, for split modes,
 * lo[i] = round(src[i] - hi[i]) in the mode's 16-bit format (lo may be NULL otherwise).
 * Replaces the cast-and-cache of kernelforge/optimized.py:186-214. */
int kf_split(const float* src, int64_t n, int mode, void* hi, void* lo, void* stream);

/* C[M, N] = act(A[M, K] . W[N, K]^T + bias[N]), output cast to c_dtype.
 * Replaces the F.linear / F.gelu / .to() sequence of kernelforge/optimized.py:441-446,
 * 483, 572-574 (cuBLAS through F.linear in the reference).
 * A is a_dtype (KF_F32, or the mode's 16-bit type, or its X2 planes with a_lo) with row
 * stride lda; W is given as planes made by kf_split for `mode` (KF_MMA_F32: w_hi is the
 * fp32 weight, w_lo unused) with row stride ldw; bias is fp32 [N] or NULL; C may be
 * KF_F32 / KF_F16 / KF_BF16 or X2 planes (c_lo). Requires K % 8 == 0, N % 4 == 0 and
 * 16-byte aligned rows. */
int kf_gemm(const void* a, const void* a_lo, int a_dtype, int64_t lda,
            const void* w_hi, const void* w_lo, int64_t ldw,
            const float* bias,
            void* c, void* c_lo, int c_dtype, int64_t ldc,
            int64_t M, int64_t N, int64_t K, int mode, int act, void* stream);

/* kf_gemm with an explicit tile (`tile` 0 = the automatic choice of kf_gemm; ids and
 * their shapes from kf_gemm_tile_info). Stateless: the choice applies to this call only,
 * and a tile that does not fit the operands (LDS-DMA tiles need 16-bit A and K a multiple
 * of their BK) falls back to the automatic one. Every tile gives bit-identical results.
 * The reference has no counterpart (cuBLAS picks its own kernel); this is the per-shape
 * tile knob of its dispatch table, `Plan.flash_block`'s GEMM analogue, for sweeps. */
int kf_gemm_tiled(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                  const void* w_hi, const void* w_lo, int64_t ldw,
                  const float* bias,
                  void* c, void* c_lo, int c_dtype, int64_t ldc,
                  int64_t M, int64_t N, int64_t K, int mode, int act, int tile, void* stream);

/* Shape of GEMM tile id `tile` (0 .. the last id; KF_EINVAL beyond): info[0..5] =
 * BM, BN, BK, LDS stages, wavefronts per block, 1 for the LDS-DMA kernel. Host only. */
int kf_gemm_tile_info(int tile, int* info);

/* Per-sequence key extent of a [B, S] validity mask: kv_len[b] = 1 + the last valid
 * position (0 if none), prefix[b] = 1 when positions [0, kv_len[b]) are all valid.
 * Prepares kf_flash_fwd's skip of fully padded key/query blocks (the reference applies
 * the key mask per block with no skip: kernelforge/ops/flash.py:159-164). */
int kf_mask_prep(const void* keep, int keep_dtype, int64_t ld_keep, int64_t B, int64_t S,
                 int32_t* kv_len, int32_t* prefix, void* stream);

/* Fused QKV projection writing the attention operand layout (the "attention layout"):
 * with d = H * hd and rows m = b * S + s of A [M = B * S, d],
 *   q_out [M, d] fp32                 = (A . Wq^T + bq)      (token-major, i.e. [B, S, H, hd])
 *   k     [M, d] 16-bit planes        = (A . Wk^T + bk)      (k_hi, k_lo; lo only for *X3)
 *   v^T   [B, H, hd, sp] 16-bit planes = (A . Wv^T + bv)^T   (keys contiguous, sp >= S, sp % 8 == 0;
 *                                       columns [S, sp) are not written: zero them for kf_flash_fwd)
 * W is the concatenated [3d, d] weight from kf_split, bias the concatenated [3d] fp32 bias.
 * Replaces the fused QKV F.linear and the strided q/k/v views of
 * kernelforge/optimized.py:483-489; writing K split and V transposed here is what lets
 * attention stage its tiles without conversion. Modes: the four 16-bit modes and
 * KF_MMA_F16X2 (which writes split planes). In KF_MMA_F16X3 / KF_MMA_BF16X3 with k_lo and
 * vt_lo both NULL, k and v^T are written as one plane each, the fp32 values rounded to
 * nearest (the operands of a single-pass attention on a split-precision projection). */
int kf_gemm_qkv(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                const void* w_hi, const void* w_lo, int64_t ldw, const float* bias,
                float* q_out, void* k_hi, void* k_lo, void* vt_hi, void* vt_lo, int64_t sp,
                int64_t B, int64_t S, int64_t H, int64_t hd, int mode, void* stream);

/* kf_gemm_qkv with an explicit tile, as kf_gemm_tiled. */
int kf_gemm_qkv_tiled(const void* a, const void* a_lo, int a_dtype, int64_t lda,
                      const void* w_hi, const void* w_lo, int64_t ldw, const float* bias,
                      float* q_out, void* k_hi, void* k_lo, void* vt_hi, void* vt_lo, int64_t sp,
                      int64_t B, int64_t S, int64_t H, int64_t hd, int mode, int tile,
                      void* stream);

/* k, v [B, H, S, hd] (strides[4] in elements, unit hd stride; fp32 / fp16 / bf16) into the
 * attention layout of kf_flash_fwd for `mode`: K planes with strides ko_strides (b, h, s, 1)
 * and V^T planes with strides vt_strides (b, h, d, 1), whose columns [S, roundup(S, 8)) it
 * zeroes (the row stride must cover them). Used when attention is called on arbitrary
 * q, k, v (the reference's flash_attention signature). k and k_hi both NULL: only V^T is
 * written (for a K that already is the mode's 16-bit type with 16-byte aligned rows, which
 * kf_flash_fwd then reads in place). */
int kf_attn_prep(const void* k, const int64_t* k_strides, const void* v, const int64_t* v_strides,
                 int in_dtype, void* k_hi, void* k_lo, const int64_t* ko_strides,
                 void* vt_hi, void* vt_lo, const int64_t* vt_strides,
                 int64_t B, int64_t H, int64_t S, int64_t hd, int mode, void* stream);

/* Host-only: the tile kf_flash_fwd uses at head_dim `hd` (8 ... 256) in MFMA `mode` (a
 * 16-bit mode): info[0..5] = BLOCK_M (query rows per block), BLOCK_N (keys per LDS
 * stage), wavefronts per block, LDS stages, 16-row query groups per wavefront, LDS bytes
 * per block. Replaces the tile-legality tables of kernelforge/ops/flash.py:277-360
 * (CANDIDATE_BLOCKS / smem_bytes / legal_blocks / pick_block), which size NVIDIA shared
 * memory; launches nothing. */
int kf_flash_tile_info(int hd, int mode, int* info);

/* Host-only check hook (no reference counterpart; launches nothing): writes
 * out[3 i .. 3 i + 2] = (batch row, head, query block) of attention block i, for every
 * block i < B * H * nqb of kf_flash_fwd's grid, as its kernels map them (XCD-contiguous
 * ranges, light/heavy causal pairs). For CPU tests of the map's bijectivity and per-XCD
 * balance; `out` holds 3 * B * H * nqb ints. */
int kf_flash_block_map(int B, int H, int nqb, int causal, int* out);

/* FlashAttention forward with causal and key-padding masks applied in registers.
 * Replaces kernelforge/ops/flash.py:363-422 (flash_attention) and its kernel :42-249.
 * q: [B, H, S, hd] view (q_strides b, h, s, 1) in fp32 / fp16 / bf16. k: 16-bit planes
 * (k_hi, k_lo for *X3 modes) with k_strides (b, h, s, 1); v: V^T planes (vt_hi, vt_lo) with
 * vt_strides (b, h, d, 1), keys contiguous, row stride >= roundup(S, 8) and columns
 * [S, roundup(S, 8)) finite -- the layout kf_gemm_qkv / kf_attn_prep write.
 * o: [B, H, S, hd] view (o_strides) in o_dtype, X2 planes allowed (o_lo). keep: [B, S]
 * (row stride ld_keep) or NULL; kv_len/prefix from kf_mask_prep (or NULL: every key is
 * scanned and keep applied everywhere). hd in {8, 16, 32, 64, 128, 256}; hd < 32 is
 * zero-padded into the MFMA contraction. softmax(q k^T * sm_scale) with fp32 online
 * accumulation; rows with no valid key produce zeros. `mode` (a 16-bit MFMA mode) is the
 * precision of both products. */
int kf_flash_fwd(const void* q, const int64_t* q_strides, int q_dtype,
                 const void* k_hi, const void* k_lo, const int64_t* k_strides,
                 const void* vt_hi, const void* vt_lo, const int64_t* vt_strides,
                 void* o, void* o_lo, const int64_t* o_strides, int o_dtype,
                 const void* keep, int keep_dtype, int64_t ld_keep,
                 const int32_t* kv_len, const int32_t* prefix,
                 int64_t B, int64_t H, int64_t S, int64_t hd,
                 float sm_scale, int mode, int flags, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Attention on arbitrary q, k, v -- kf_attn_prep, then kf_mask_prep when `keep` is given,
 * then kf_flash_fwd, with the same arguments and results -- but with the K / V^T planes
 * and kv_len / prefix staged in a static device buffer of the library (64 MiB per GPU,
 * held until the process ends) instead of caller buffers: it allocates nothing. q, k, v
 * are [B, H, S, hd] views (strides[4], unit hd stride) of `in_dtype`; o as kf_flash_fwd.
 * Rejects (KF_EINVAL, nothing launched) a problem whose staging exceeds the buffer:
 * (2 B * 4 bytes if keep) + planes * 2 bytes * B * H * hd * (S + roundup(S, 8)), each
 * piece rounded up to 256 bytes, planes = 2 for *X3 modes, else 1. Every call on one GPU
 * uses the same buffer: calls that overlap on one GPU race. */
int kf_flash_attention_static(const void* q, const int64_t* q_strides,
                              const void* k, const int64_t* k_strides,
                              const void* v, const int64_t* v_strides, int in_dtype,
                              void* o, void* o_lo, const int64_t* o_strides, int o_dtype,
                              const void* keep, int keep_dtype, int64_t ld_keep,
                              int64_t B, int64_t H, int64_t S, int64_t hd,
                              float sm_scale, int mode, int flags, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KF950_H */
