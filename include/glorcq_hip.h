/*
 * glorcq_hip.h — C ABI of the MI355X (gfx950) GLoRCQ hot-path library.
 *
 * The library computes the fused "dequantize + GEMV/GEMM + low-rank
 * correction" that a GLoRCQ quantized linear layer runs for every projection:
 *
 *     y[m, n] = sum_k W[n, k] * x[m, k]  +  sum_j a[m, j] * SV[n, j]  + bias[n]
 *     W[n, k] = s[n, k/g] * (q[n, k] - z[n, k/g])       (asymmetric, sym = 0)
 *     W[n, k] = s[n, k/g] * q_signed[n, k]              (symmetric, sym = 1)
 *     W[n, k] = s[n, k/g] * (q_signed[n, k] - z[n, k/g])   (signed asymmetric, sym = 2)
 *     a[m, j] = sum_k x[m, k] * U[k, j]                 (or a caller-supplied a)
 *
 * Data format (device memory, all row-major, little-endian):
 *   codes   int32 (N, K*bits/32): b-bit codes packed LSB-first along K; code k
 *           of row n sits in word k/(32/b) at bit offset b*(k % (32/b)).
 *           sym = 0: unsigned codes 0..2^b-1.  sym = 1: b-bit two's
 *           complement.  sym = 2: signed codes -2^(b-1)..2^(b-1)-1 stored
 *           as q + 2^(b-1) (two's complement with the sign bit flipped), so
 *           that z stays exact in fp16 (the reference's int8 codes with
 *           non-integer zero-points, gptq_matmul.cu:15-16).
 *   scales  fp16 (N, K/g)     zeros fp16 (N, K/g) (ignored when sym == 1)
 *   U       fp16 (K, r)       input-side low-rank factor (shared per cluster)
 *   SV      fp16 (N, r)       output-side low-rank factor with S fused in
 *   x       fp16 (M, K)       y fp16 (M, N)      bias fp16 (N) or NULL
 *
 * Reference interface replaced (nicyyyy/GLoRCQ):
 *   inference/kernels/__init__.py:284-346  gptq_dequant_matmul_fused
 *   inference/kernels/gptq_matmul.cu:223-315 gptq_dequant_matmul_cuda (host)
 *   inference/quantized_linear.py:286-355   GLoRCQLinear.forward (+ LoRA add)
 *
 * Conventions: every pointer argument is a device pointer unless stated; every
 * entry point launches on the given HIP stream (`stream`, a hipStream_t passed
 * as void*; NULL = default stream), never synchronizes, never allocates device
 * memory, and returns 0 on success or a nonzero GLQ_ERR_* code.  The message
 * of the last failure on the calling thread is available from
 * glq_last_error().  Empty work (M == 0 or N == 0) is a successful no-op.
 */
#ifndef GLORCQ_HIP_H
#define GLORCQ_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLQ_OK 0
#define GLQ_ERR_INVALID 1   /* argument check failed (the TORCH_CHECK analogue) */
#define GLQ_ERR_HIP 2       /* a HIP runtime call or kernel launch failed       */

/* Library version (major*10000 + minor*100 + patch). */
int glq_version(void);

/* Message of the last error raised on the calling thread ("" if none). */
const char* glq_last_error(void);

/*
 * Bytes of workspace glq_gemv_lora / glq_gemv_lora_batched need for `items`
 * independent problems of shape (M, K, N, rank) when they compute a = x U
 * themselves (0 when rank == 0).  Its first 69632 bytes are arrival
 * counters (4096 bytes) and the one-token-row launch's x U words (64 KiB):
 * the 4..16-row token-tile launch forms a = x U in its own first workgroups
 * and hands it to the rest, and the one-row launch has jobs in front of its
 * grid form K-slice sums of a that its row workgroups read.  They must be
 * zero before the workspace's first use with these entry points (allocate
 * it zero-filled), every call leaves them zero, and the buffer must serve no
 * other entry point.  The rest holds fp32 partial sums of a over K-slices of U and needs
 * no initialisation.  Calls that may run concurrently (different streams)
 * need different workspaces.
 */
int64_t glq_gemv_workspace_bytes(int64_t items, int64_t M, int64_t K,
                                 int64_t N, int64_t rank);

/*
 * Fused dequant-GEMV + low-rank correction, 1 <= M <= 16 (decode).
 * Replaces gptq_dequant_matmul_fused (inference/kernels/__init__.py:284) and
 * the LoRA tail of GLoRCQLinear.forward (inference/quantized_linear.py:338-349).
 *   bits      2 or 4;  K % group == 0;  group % 128 == 0, or any group of
 *             whole 16-byte pieces (a multiple of 128/bits codes) when a
 *             code row has at most 128 pieces and rank <= 128 (one lane-
 *             kernel launch per token row: the reference's 64 x 64, group
 *             64 case, test_gptq_kernel.py:193)
 *   sym       0, 1 or 2 (code formats above)
 *   U, SV     may be NULL (no correction) ; rank % 8 == 0, rank <= 512
 *   xU        optional precomputed a = x*U (M, rank) fp16 (cluster-shared
 *             x*U, the `precomputed_xU` hook of quantized_linear.py:286); when
 *             given, U is not read.
 *   bias      optional (N) fp16
 *   workspace device buffer of glq_gemv_workspace_bytes(1, M, K, N, rank),
 *             256-byte aligned (may be NULL when xU is given or rank == 0)
 * Launches: M == 1 (code rows of at most 128 16-byte pieces): one, whose
 * workgroups form a = x*U, the GEMV and a*SV^T; 4..16 rows of 4-bit codes
 * (the token-tile form): one, whose first workgroups form a = x*U and hand it
 * to the row blocks' stores; otherwise a K-sliced x*U partial-sum kernel
 * (only when U is used), then the GEMV kernel, whose epilogue adds a*SV^T
 * and rounds once to fp16.
 */
int glq_gemv_lora(const void* x, int64_t M, int64_t K, int64_t N,
                  const int32_t* codes, int bits, const void* scales,
                  const void* zeros, int64_t group, int sym, const void* U,
                  const void* SV, int64_t rank, const void* xU,
                  const void* bias, void* y, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * Allocation-free form of glq_gemv_lora.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory or pass a
 * workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as glq_gemv_lora,
 * without the workspace: the x*U partials go to a static per-GPU scratch
 * array of glq_gemv_noalloc_max_scratch_bytes() bytes (4 MiB) inside the
 * library, so calls needing more (glq_gemv_workspace_bytes(1, M, K, N, rank)
 * when U is used) fail with GLQ_ERR_INVALID.  Every call on one GPU shares
 * that GPU's scratch: calls that may overlap on one GPU (different streams,
 * or different host threads) race and must be ordered by the caller.  The
 * scratch's header (counter words and the one-row launch's x*U words) starts
 * at zero (static device memory) and every call leaves it zero; the partials
 * are fully rewritten by each call.
 */
int64_t glq_gemv_noalloc_max_scratch_bytes(void);
int glq_gemv_lora_noalloc(const void* x, int64_t M, int64_t K, int64_t N,
                          const int32_t* codes, int bits, const void* scales,
                          const void* zeros, int64_t group, int sym, const void* U,
                          const void* SV, int64_t rank, const void* xU,
                          const void* bias, void* y, void* stream);

/*
 * Batched form: `items` independent problems of one shape in ONE launch, item
 * i reading codes + i*codes_stride (int32 elements), scales/zeros + i*sz_stride,
 * U + i*u_stride, SV + i*sv_stride, bias + i*bias_stride, x + i*x_stride,
 * xU + i*xu_stride and writing y + i*y_stride (fp16 elements).  This is the
 * grouped expert GEMV of the reference's graph-mode MoE step
 * (turbo_dequant_grouped_gemv, inference/kernels/__init__.py:242-278), in the
 * packed group-quantized format.
 */
int glq_gemv_lora_batched(int64_t items, const void* x, int64_t x_stride,
                          int64_t M, int64_t K, int64_t N,
                          const int32_t* codes, int64_t codes_stride, int bits,
                          const void* scales, const void* zeros,
                          int64_t sz_stride, int64_t group, int sym,
                          const void* U, int64_t u_stride, const void* SV,
                          int64_t sv_stride, int64_t rank, const void* xU,
                          int64_t xu_stride, const void* bias,
                          int64_t bias_stride, void* y, int64_t y_stride,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

/*
 * Batched form with cluster-shared U: item i reads U + u_index[i]*u_stride
 * (u_index: `items` int32 on the device, each clamped to [0, n_u)), so one
 * copy of a cluster's U serves every item of the cluster.  This is the
 * reference's per-cluster U shared by the cluster's experts
 * (_precompute_xU_for_experts, inference/moe_block.py:290-322; the same
 * cluster fusion in _batched_proj_forward, moe_block.py:545-565), and it
 * serves projections that share an input and a U (q, k and v of one layer
 * cut into equal items).  Other arguments as glq_gemv_lora_batched;
 * u_index is required.  xU, when not NULL, is a = x U given per U matrix
 * ((n_u, M, rank) fp16 at xu_stride halves apart, item i reading row block
 * u_index[i]) and U is then not read.
 */
int glq_gemv_lora_clustered(int64_t items, const void* x, int64_t x_stride,
                            int64_t M, int64_t K, int64_t N,
                            const int32_t* codes, int64_t codes_stride, int bits,
                            const void* scales, const void* zeros,
                            int64_t sz_stride, int64_t group, int sym,
                            const void* U, int64_t u_stride,
                            const int32_t* u_index, int64_t n_u, const void* xU,
                            int64_t xu_stride, const void* SV,
                            int64_t sv_stride, int64_t rank, const void* bias,
                            int64_t bias_stride, void* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes,
                            void* stream);

/*
 * Batched GEMV whose a = x U arrives as fp32 partials: item i takes
 *   a[m][j] = fp16(parts[b][0][m][j] + parts[b][1][m][j] + ... + parts[b][P-1][m][j])
 * (summed in that order), b = u_index[i] (clamped to [0, n_u)) or b = i
 * when u_index is NULL; parts is (blocks, P, M, rpad) fp32 with rpad = rank
 * rounded up to 32 -- what glq_rmsnorm_xu and glq_decode_attention_xu write,
 * so the projection after a norm or an attention launch streams its codes
 * with no x U launch or x U work of its own.  The reference's fused forward
 * with a precomputed a (GLoRCQLinear.forward with precomputed_xU,
 * inference/quantized_linear.py:338-345).  Other arguments as
 * glq_gemv_lora_batched (no U, no workspace); M > 1 takes whole 128-code
 * groups.
 */
int glq_gemv_lora_parts(int64_t items, const void* x, int64_t x_stride, int64_t M, int64_t K,
                        int64_t N, const int32_t* codes, int64_t codes_stride, int bits,
                        const void* scales, const void* zeros, int64_t sz_stride, int64_t group,
                        int sym, const void* SV, int64_t sv_stride, int64_t rank,
                        const float* parts, int64_t P, const int32_t* u_index, int64_t n_u,
                        const void* bias, int64_t bias_stride, void* y, int64_t y_stride,
                        void* stream);

/*
 * Low-rank factor a = fp16(x U) for `items` problems: x (M, K) fp16 at
 * x + i*x_stride, U (K, rank) fp16 at U + i*u_stride, a (M, rank) fp16
 * written at xu + i*xu_stride (fp32 accumulation, one rounding).  This is the
 * reference's `x @ U` (inference/quantized_linear.py:344) and the
 * cluster-shared precompute `_precompute_xU_for_experts`
 * (inference/moe_block.py:290-322): pass x_stride = 0 to apply one x to
 * several clusters' U.  Two launches: K-sliced fp32 partial sums into the
 * workspace (glq_lowrank_workspace_bytes), then a summing kernel.  Feed the
 * result to glq_gemv_lora*(xU=...).
 */
int64_t glq_lowrank_workspace_bytes(int64_t items, int64_t M, int64_t K, int64_t rank);
int glq_lowrank_xu_batched(int64_t items, const void* x, int64_t x_stride, int64_t M, int64_t K,
                           const void* U, int64_t u_stride, int64_t rank, void* xu,
                           int64_t xu_stride, void* workspace, int64_t workspace_bytes,
                           void* stream);
/*
 * The same for the picks of a MoE step: a[p] = fp16(x[p] U_c) (x (picks, K)
 * fp16, a (picks, rank) fp16) with U_c row c = cluster_of[sel[p]] of U
 * (u_rows, K, rank) -- each routed expert's down projection's own
 * a = fp16(inter @ U_down) (inference/moe_block.py:661-676).  sel values are
 * clamped into [0, experts), cluster_of values into [0, u_rows).  Workspace:
 * glq_lowrank_workspace_bytes(picks, 1, K, rank).
 */
int glq_lowrank_xu_routed(int64_t picks, const void* x, int64_t K, const void* U,
                          int64_t u_rows, int64_t rank, const int32_t* sel, int64_t experts,
                          const int32_t* cluster_of, void* xu, void* workspace,
                          int64_t workspace_bytes, void* stream);

/*
 * Prefill GEMM (any M, built for M > 16): y = dequant(codes) x + (x U) SV^T
 * + bias with the same arguments and results as glq_gemv_lora.  Replaces the
 * reference's gptq_dequant_gemm_kernel path (inference/kernels/gptq_matmul.cu:
 * 111-213, taken for B > 4) and the LoRA tail of GLoRCQLinear.forward
 * (inference/quantized_linear.py:338-349).  Group 128.  Codes decode into
 * exact fp16 operands (q - zero-point's integer part) of
 * v_mfma_f32_16x16x32_f16, each group's fp32 sum scaled once (any zero-point,
 * symmetric or not); a = fp16(x U) comes from xU or from a low-rank launch
 * before the GEMM (rank <= 128: one launch whose 16-row blocks' K slices
 * hand their partial sums to the block's last arriving slice).
 * The workspace (glq_gemm_workspace_bytes, 256-byte aligned) is required.
 * When U is given (no xU) its first 4096 bytes are arrival counters: they
 * must be zero before the workspace's first use with glq_gemm_lora (allocate
 * it zero-filled) and every call leaves them zero; do not share the buffer
 * with other entry points.  The rest needs no initialisation.
 */
int64_t glq_gemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int64_t rank);
int glq_gemm_lora(const void* x, int64_t M, int64_t K, int64_t N,
                  const int32_t* codes, int bits, const void* scales,
                  const void* zeros, int64_t group, int sym,
                  const void* U, const void* SV, int64_t rank, const void* xU,
                  const void* bias, void* y, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * TurboQuant codebook matmul, for `items` independent problems:
 *   y[i][m][n] = fp16(norms[i][n] * sum_k C[q_i(n, k)] * x_rot[i][m][k])
 * Replaces the reference's turbo_dequant_matmul op (inference/kernels/
 * turbo_matmul.cu:255-318 host; turbo_dequant_gemv_2bit_kernel :46-137 for
 * B <= 4, turbo_dequant_gemm_2bit_kernel :150-245 otherwise; registered as
 * glorcq::turbo_dequant_matmul, inference/kernels/__init__.py:68-85) with
 * items = 1, and the grouped op turbo_dequant_grouped_gemv (turbo_matmul.cu:
 * 417-464, kernel :329-415) with items = E, M = 1 and per-item strides.
 *   x_rot   (items, M, K) fp16, item stride x_stride elements (0: shared)
 *   codes   2-bit indices, (items, N, K/16) int32 words = the reference's
 *           packed_indices (N, K/4) uint8 (4 per byte, LSB-first) read as
 *           little-endian words; item stride codes_stride words
 *   norms   (items, N) fp32, item stride norms_stride
 *   centroids (4,) fp32 codebook
 *   xU, SV  optional low-rank term + a SV^T: a = fp16(x U) (items, M, rank)
 *           from glq_lowrank_xu_batched on the UNrotated x, SV (items, N,
 *           rank); rank a multiple of 8 <= 256.  SV == NULL or rank 0: none.
 *           This is GLoRCQLinear.forward's LoRA tail for turbo layers
 *           (inference/quantized_linear.py:338-349) and lora_USV of
 *           turbo_dequant_matmul_fused (inference/kernels/__init__.py:234-237)
 *   bias    optional (items, N) fp16
 *   y       (items, M, N) fp16 = fp16(norm * acc + a SV^T + bias), item
 *           stride y_stride
 * K must be a multiple of 64; x_rot and codes 16-byte aligned.  Any M.
 */
int glq_turbo_gemv_batched(int64_t items, const void* x_rot, int64_t x_stride,
                           int64_t M, int64_t K, int64_t N, const int32_t* codes,
                           int64_t codes_stride, const float* norms,
                           int64_t norms_stride, const float* centroids,
                           const void* xU, int64_t xu_stride, const void* SV,
                           int64_t sv_stride, int64_t rank, const void* bias,
                           int64_t bias_stride, void* y, int64_t y_stride,
                           void* stream);

/*
 * Randomized Hadamard transform of `rows` rows of length d (a power of two
 * <= 32768), H the Sylvester Hadamard matrix, fp32 arithmetic:
 *   inverse == 0: y = (1/sqrt(d)) H diag(signs) x   (rht_forward,
 *                 hadamard_rotation.py:52-67)
 *   inverse != 0: y = diag(signs) (1/sqrt(d)) H x   (rht_backward, :70-86)
 * x and y are fp16 (flag 0) or fp32 (flag 1); the hot-path call
 * rht_forward(x.float(), signs).half() (inference/moe_block.py:351,525,649,
 * 840) is x_fp32 = y_fp32 = 0.  The reference relies on the external
 * fast-hadamard-transform package for H.  signs: (d,) fp32 of +-1.  y may not
 * alias x.
 */
int glq_rht(const void* x, int x_fp32, int64_t rows, int64_t d, const float* signs,
            int inverse, void* y, int y_fp32, void* stream);

/*
 * Load-time dequantization of an intN LoRA factor (U or SV) to fp16:
 *   out[r][c] = fp16((q[r][c] / (2^(nbits-1) - 1)) * scale)   (fp32 math)
 * q is int8 (rows, cols) (int4_packed == 0), or uint8 ((rows+1)/2, cols)
 * holding row pairs in nibbles (row 2i low, row 2i+1 high, value - 7;
 * int4_packed != 0, nbits 4).  scale is fp16 per column (cols,) or, with
 * scale_per_row, per row (rows, 1).  Replaces _dequant_intN and _unpack_int4
 * (inference/model_builder.py:69-80) as used by SharedUCache (:27-66) and
 * _load_lora_for_module (:465-544); bit-identical to their fp32 arithmetic
 * followed by .half().
 */
int glq_dequant_factor(const void* q, int int4_packed, int64_t rows, int64_t cols,
                       const void* scale, int scale_per_row, int nbits, void* out,
                       void* stream);

/*
 * One MoE block at decode: router, top-k dispatch, routed SwiGLU experts with
 * cluster-shared low-rank correction, sigmoid-gated shared expert, combine.
 * Replaces GraphCompatibleMoeBlock.forward (inference/moe_block.py:381-436:
 * router :386-392, cluster-shared x*U :290-322, per-expert
 * down(act(gate(x)) * up(x)) with LoRA :367-379 and :438-478, shared expert
 * :429-433) and the HF-style GLoRCQExperts.forward
 * (inference/quantized_linear.py:395-428) for one step of `tokens` tokens.
 * Only selected experts are read (the reference's graph mode computes all E,
 * moe_block.py:742-890).  All routing stays on the device: no host sync, so
 * the call can be captured in a hipGraph (graph_wrapper.py:69-131).
 *
 * Weights are stacked expert-major; projection index 0 = gate, 1 = up,
 * 2 = down.  gate/up: N = inter, K = hidden; down: N = hidden, K = inter.
 * Codes use the packed container of glq_gemv_lora (bits 2 or 4, group 128,
 * asymmetric: zeros required).  U is the per-projection cluster pool
 * (the reference's global U pool, model_builder.py:143-183); an expert's U is
 * U[cluster_of[e]].  rank 0 or SV == NULL: no low-rank term.
 */
typedef struct glq_moe_params {
  int64_t tokens;        /* B: rows of h (1..64) */
  int64_t hidden;        /* H */
  int64_t experts;       /* E (<= 256) */
  int64_t inter;         /* routed expert intermediate size */
  int64_t top_k;         /* <= 16, tokens * top_k <= 512 */
  int64_t n_clusters;    /* U clusters per projection */
  int64_t rank;          /* LoRA rank: 0, or a multiple of 8 <= 128 */
  int64_t shared_inter;  /* shared expert intermediate size (0: no shared expert) */
  int32_t norm_topk_prob;
  int32_t bits;          /* routed code width: 2 or 4 */
  int32_t shared_bits;   /* shared expert code width: 2 or 4 */
  int32_t group;         /* quantization group: 128 */
  const void* h;                 /* (tokens, hidden) fp16 */
  const void* router_w;          /* (experts, hidden) fp16 */
  const void* shared_gate_w;     /* (hidden,) fp16; NULL: shared output ungated */
  const int32_t* codes[3];       /* (experts, N, K*bits/32) */
  const void* scales[3];         /* (experts, N, K/group) fp16 */
  const void* zeros[3];          /* (experts, N, K/group) fp16 */
  const void* U[3];              /* (n_clusters or u_rows, K, rank) fp16 */
  const int32_t* cluster_of[3];  /* (experts,) int32 */
  const void* SV[3];             /* (experts, N, rank) fp16 */
  const int32_t* shared_codes[3];  /* (N, K*shared_bits/32) */
  const void* shared_scales[3];    /* (N, K/group) fp16 */
  const void* shared_zeros[3];
  void* out;             /* (tokens, hidden) fp16 */
  void* router_logits;   /* (tokens, experts) fp16, or NULL */
  /* Cross-layer U pool (the reference's global U pool, model_builder.py:
   * 143-183): U[s] may hold more rows than this block's clusters.
   * u_slot[s] (s = gate, up): (n_clusters,) int32 row of U[s] holding
   * cluster c's factor, or NULL (row = c).  For down, cluster_of[2][e] is the
   * row of U[2] directly.  u_rows[s]: rows of U[s] (0: n_clusters). */
  const int32_t* u_slot[2];
  int64_t u_rows[3];
  /* (tokens, hidden) fp16 or NULL: out = fp16(residual + fp16(block output)),
   * the decoder layer's residual add after the MoE block. */
  const void* residual;
} glq_moe_params;

/* Workspace bytes glq_moe_decode needs for `p` (negative on a bad shape). */
int64_t glq_moe_workspace_bytes(const glq_moe_params* p);
/*
 * Four launches on `stream` (five when the x*U jobs are gated on routing);
 * a step of 17-32 tokens with at most 4 per expert on average runs as
 * consecutive steps of at most 16 tokens.
 * The workspace (256-byte aligned) must be zero-filled before its first use:
 * its first 8192 bytes hold arrival counters (router workgroups, the
 * combine's and the token-tile form's row blocks, the a_down word), and
 * every step leaves them zero again.  Steps that share a workspace must not
 * overlap.
 */
int glq_moe_decode(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                   void* stream);

/*
 * One MoE block over many tokens (a prompt): the reference's _forward_sparse
 * (inference/moe_block.py:704-740) -- every active expert's SwiGLU
 * projections on its gathered tokens -- with the same params as
 * glq_moe_decode and the decode step's routing and combine arithmetic.
 * tokens up to 2^20; routed and shared-expert codes must use integer
 * zero-points (GPTQ zero-points are integers; the kernels use round(z), so
 * run glq_moe_decode steps otherwise).  Launches:
 * router (+ x in the GEMMs' decode order), dispatch (pairs sorted by expert,
 * token tiles), the low-rank a = x U per pair, the grouped gate/up GEMM with
 * SwiGLU, the low-rank a of the down input, the grouped down GEMM, the
 * shared expert's two GEMMs, the combine.  The workspace (256-byte aligned,
 * glq_moe_prefill_workspace_bytes) needs no initialisation.
 */
int64_t glq_moe_prefill_workspace_bytes(const glq_moe_params* p);
int glq_moe_prefill(const glq_moe_params* p, void* workspace, int64_t workspace_bytes,
                    void* stream);

/*
 * The pieces of a decode step whose routed experts are TurboQuant layers
 * (the reference's 2-bit expert format; inference/moe_block.py:381-436 with
 * the turbo expert projections of :480-702), composed by
 * glorcq_amd/moe_block.py.  Picks are p = t * top_k + k.
 *
 * glq_moe_route: the router of glq_moe_decode alone (moe_block.py:386-392):
 * fp16 logits, fp32 softmax, top-k (ties to the lower index), optional
 * renormalisation, weights rounded to fp16; sel (tokens * top_k) int32,
 * weights (tokens * top_k) fp16, shared_gate (tokens) fp16 =
 * sigmoid(h . shared_gate_w) (1 when shared_gate_w is NULL), logits (tokens,
 * experts) fp16 or NULL.  hidden a multiple of 8, <= 4096.  The workspace
 * (glq_moe_route_workspace_bytes, 16-byte aligned) must be zero-filled before
 * its first use; every call leaves its counters zero.
 */
int64_t glq_moe_route_workspace_bytes(int64_t tokens, int64_t experts);
int glq_moe_route(const void* h, const void* router_w, const void* shared_gate_w,
                  int64_t tokens, int64_t hidden, int64_t experts, int64_t top_k,
                  int norm_topk_prob, int32_t* sel, void* weights, void* shared_gate,
                  void* logits, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * A GPTQ shared expert riding in the launches of a TurboQuant block's decode
 * step (glq_turbo_moe_prep: gate and up, glq_turbo_moe_down_prep: down):
 * codes/scales/zeros of gate, up, down as in glq_moe_params (unsigned codes
 * with zero-points, group 128), inter its width, bits 2 or 4.
 *   sinter (tokens, inter) fp16 = fp16(fp16(silu(fp16(h gate^T))) * fp16(h up^T))
 *   sy (tokens, hidden) fp16 = fp16(sinter down^T), the shared expert's
 *   output for glq_moe_combine (moe_block.py:429-435).
 */
typedef struct glq_moe_shared {
  const int32_t* codes[3];
  const void* scales[3];
  const void* zeros[3];
  int64_t inter;
  int32_t bits;
  int32_t reserved;
  void* sinter;
  void* sy;
} glq_moe_shared;

/*
 * The first launch of a TurboQuant block's decode step (the composition in
 * glorcq_amd/moe_block.py): glq_moe_route's routing (same arguments,
 * outputs and workspace contract), and in the same launch, from the same h:
 * with rht_signs, x_rot = fp16((1/sqrt(hidden)) H diag(rht_signs) h) for
 * gate and up (rht_forward(h.float(), signs).half(),
 * inference/moe_block.py:351; hidden a power of two); with n_u > 0, the
 * fp32 partials of h U_u over 256-row slices for the n_u matrices U
 * (n_u, hidden, rank) -- every gate and up cluster's x U,
 * _precompute_xU_for_experts (moe_block.py:290-322) -- into parts
 * (n_u, S, tokens, rpad), S = ceil(hidden / 256), rpad = rank rounded up
 * to 32, which glq_turbo_moe_gemv2 sums in slice order; with shared, the
 * shared expert's gate and up rows (sinter).  tokens <= 16.
 */
int glq_turbo_moe_prep(const void* h, const void* router_w, const void* shared_gate_w,
                       int64_t tokens, int64_t hidden, int64_t experts, int64_t top_k,
                       int norm_topk_prob, int32_t* sel, void* weights, void* shared_gate,
                       void* logits, void* workspace, int64_t workspace_bytes,
                       const float* rht_signs, void* x_rot, const void* U, int64_t n_u,
                       int64_t rank, float* parts, const glq_moe_shared* shared,
                       void* stream);

/* One projection of the TurboQuant experts for glq_turbo_moe_gemv2. */
typedef struct glq_turbo_mat {
  const void* x_rot;      /* the rotated input: row p / x_div for pick p, K fp16 each */
  const int32_t* codes;   /* (experts, N, K/16) */
  const float* norms;     /* (experts, N) */
  const float* centroids; /* (4,) */
  const void* SV;         /* (experts, N, rank) fp16, or NULL: no low-rank term */
  const float* parts;     /* a as fp32 partials (blocks, P, rows, rpad) */
  const int32_t* cluster; /* expert -> block, row = p / x_div (rows = tokens); NULL:
                             block = pick p, rows = 1 */
  int64_t blocks;
} glq_turbo_mat;

/*
 * glq_turbo_moe_gemv with a given as partials (what glq_turbo_moe_prep
 * writes for gate and up, glq_turbo_moe_down_prep for down): pick p's a =
 * fp16(sum over s in order of parts[b][s][row]), b = cluster[sel[p]] (or
 * p), then y = fp16(norm * C[q] . x_rot + a SV^T).  With up != NULL the
 * launch walks both matrices (the same shape; gate = m) and stores the
 * SwiGLU inter fp16(fp16(silu(fp16(gate))) * fp16(up)) -- the bits of the
 * gate launch followed by the up launch's SwiGLU store, in one launch
 * (the reference's act_fn(gate) * up, moe_block.py:465-468).  y (picks, N).
 */
int glq_turbo_moe_gemv2(int64_t picks, int64_t x_div, int64_t K, int64_t N, int64_t experts,
                        const int32_t* sel, const glq_turbo_mat* m, const glq_turbo_mat* up,
                        int64_t rank, int64_t P, void* y, void* stream);

/*
 * The down projection's inputs of a TurboQuant block's decode step, in one
 * launch, for every pick p (inter (picks, inter_dim) fp16, the SwiGLU of
 * glq_turbo_moe_gemv2): xd[p] = fp16(inter[p] Pi^T) with Pi (inter_dim,
 * inter_dim) fp16 row-major (the QR rotation, moe_block.py:352-356;
 * inter_dim a multiple of 32), or with rht_signs instead the transform
 * fp16((1/sqrt(d)) H diag(signs) inter[p]) (d a power of two); and with U
 * (n_clusters, inter_dim, rank) the fp32 partials of inter[p]
 * U[cluster[sel[p]]] over 256-row slices into parts (picks, S, 1, rpad),
 * the down GEMV's a (glq_turbo_moe_gemv2 with cluster = NULL); with shared,
 * the shared expert's down rows over its sinter (tokens of hidden values,
 * sy).
 */
int glq_turbo_moe_down_prep(int64_t picks, int64_t inter_dim, const void* inter, const void* Pi,
                            const float* rht_signs, void* xd, const void* U, int64_t n_clusters,
                            const int32_t* cluster, const int32_t* sel, int64_t experts,
                            int64_t rank, float* parts, int64_t tokens, int64_t hidden,
                            const glq_moe_shared* shared, void* stream);

/*
 * Turbo GEMV of every pick (turbo_dequant_matmul_fused per expert,
 * inference/kernels/__init__.py:184-239, as _batched_proj_forward and
 * _batched_down_forward call it, moe_block.py:480-702): pick p multiplies x
 * row p / x_div of x_rot (K) by expert sel[p]'s codes (experts, N, K/16)
 * int32, norms (experts, N) fp32 and the shared centroids, plus
 * a SV_sel[p]^T with a = xU row xu_cluster[sel[p]] * xu_tokens + p / x_div
 * (xU rows clamped below xu_rows; xu_cluster NULL: row p), SV (experts, N,
 * rank), and bias (experts, N) if given.  y (picks, N) fp16; with gate
 * (picks, N) fp16 the store is fp16(fp16(silu(gate)) * fp16(y)) (the up
 * projection's launch forms the SwiGLU inter).  sel values are clamped into
 * [0, experts).
 */
int glq_turbo_moe_gemv(int64_t picks, int64_t x_div, const void* x_rot, int64_t K, int64_t N,
                       int64_t experts, const int32_t* sel, const int32_t* codes,
                       const float* norms, const float* centroids, const void* xU,
                       const int32_t* xu_cluster, int64_t xu_tokens, int64_t xu_rows,
                       const void* SV, int64_t rank, const void* bias, const void* gate,
                       void* y, void* stream);

/*
 * out[t] = fp16(sum_k weights[t][k] y[t top_k + k] + shared_gate[t] shared[t])
 * (+ residual[t]): the block's weighted sum (moe_block.py:470-476) and the
 * gated shared expert (:429-435) in fp32, rounded once (shared NULL: no
 * shared term; residual NULL: none).  y (tokens * top_k, hidden) fp16.
 */
int glq_moe_combine(const void* y, const void* weights, const void* shared,
                    const void* shared_gate, const void* residual, int64_t tokens,
                    int64_t hidden, int64_t top_k, void* out, void* stream);

/* out = fp16(fp16(silu(gate)) * up), n fp16 elements (act_fn(gate) * up,
 * moe_block.py:465-468 on a shared expert). */
int glq_swiglu(const void* gate, const void* up, int64_t n, void* out, void* stream);

/*
 * Debug: unpack codes (N, K*bits/32) int32 -> (N, K) int32.  Codes are
 * returned unsigned (0..2^b-1), or sign-extended when sym != 0.
 * Replaces _unpack_indices (inference/quantized_linear.py:115-146) and
 * _unpack_indices_2bit (inference/kernels/__init__.py:113-118) for the packed
 * int32 container.
 */
int glq_unpack_codes(const int32_t* codes, int64_t N, int64_t K, int bits,
                     int sym, int32_t* out, void* stream);

/*
 * Debug: dequantize to fp16 W (N, K), bit-exactly fp16(fp16(q - z) * s)
 * (sym: fp16(q * s)), i.e. GLoRCQLinear._dequant_gptq
 * (inference/quantized_linear.py:271-284).
 */
int glq_dequant_weight(const int32_t* codes, int64_t N, int64_t K, int bits,
                       const void* scales, const void* zeros, int64_t group,
                       int sym, void* W, void* stream);

/*
 * Packs (N, K) int32 codes into the int32 container on the device (load-time
 * helper; values are masked to b bits, so two's-complement symmetric codes
 * pack directly).  Replaces the per-call int32->int8 cast of the reference
 * (inference/kernels/__init__.py:305-309) with a one-time pack.
 */
int glq_pack_codes(const int32_t* q, int64_t N, int64_t K, int bits,
                   int32_t* codes, void* stream);

/*
 * ---- Decoder-layer pieces of the model-level decode step ----
 * The reference's model path runs these steps as framework (transformers)
 * ops around its quantized projections (inference/graph_wrapper.py:69-149
 * captures the whole step, model_builder.py:186-197 swaps only the MoE
 * blocks); it has no kernels of its own for them, so these have no
 * reference kernel counterpart.  They replace transformers' Qwen3-MoE
 * modules (modeling_qwen3_moe: Qwen3MoeRMSNorm.forward, the decoder layer's
 * residual adds, Qwen3MoeAttention.forward's q_norm / k_norm,
 * apply_rotary_pos_emb, StaticLayer.update and the scaled-dot-product
 * attention of one decode token), one launch each, with the framework's fp16
 * rounding points kept.
 */

/*
 * RMSNorm of `rows` rows of `dim` fp16 values (dim % 8 == 0, dim <= 8192):
 *   y = x, or fp16(x + residual) when residual != NULL (then written to
 *   residual_out); out = fp16(weight * fp16(y * rsqrt(mean(y^2) + eps))).
 * x, residual, weight, out, residual_out 16-byte aligned; out may alias x.
 */
int glq_rmsnorm(const void* x, const void* residual, const void* weight, int64_t rows,
                int64_t dim, float eps, void* out, void* residual_out, void* stream);

/*
 * glq_rmsnorm of rows <= 16 rows and, in the same launch, the low-rank
 * factors of the projections that read its output, as fp32 partials: for
 * each of the n_u matrices U_u (dim, rank) fp16 at U + u*u_stride and each
 * 256-row slice s of dim (S = ceil(dim / 256) slices),
 *   parts[u][s][m][j] = sum over k in slice s of out[m][k] U_u[k][j]
 * (fp32, (n_u, S, rows, rpad) with rpad = rank rounded up to 32; columns
 * past rank are zero).  glq_gemv_lora_parts sums them in slice order as its
 * a, so the projections of a decoder layer's attention (q, k, v after the
 * input RMSNorm) stream their codes with no x U of their own.  No reference
 * kernel: the reference forms x U inside each GLoRCQLinear.forward
 * (inference/quantized_linear.py:338-345) after the framework's RMSNorm.
 * out and residual_out carry the same bits as glq_rmsnorm's.  rank a
 * multiple of 8 (<= 1024), n_u <= 65535; no workspace.
 */
int glq_rmsnorm_xu(const void* x, const void* residual, const void* weight, int64_t rows,
                   int64_t dim, float eps, void* out, void* residual_out, const void* U,
                   int64_t u_stride, int64_t n_u, int64_t rank, float* parts, void* stream);

/*
 * One decode token per row (tokens rows): per-head RMSNorm of q (q_heads
 * heads) and k (kv_heads heads) over head_dim = 128 with weights q_norm_w /
 * k_norm_w, then the rotary embedding x' = fp16(fp16(x cos) +
 * fp16(rotate_half(x) sin)) with cos/sin rows of 128 fp16 (cs_stride values
 * apart; 0 = one row for all tokens).  q' goes to q_out (tokens, q_heads,
 * 128); k' and v (unchanged) to the static caches (tokens, kv_heads, max_len,
 * 128) at position *pos (device int64; out-of-range positions write
 * nothing), and *pos + 1 to *len_out (device int32) for
 * glq_decode_attention.  q, k, v rows are q_stride / kv_stride values apart;
 * with q_item_rows > 0, q is instead item-major (q_heads * 128 / q_item_rows,
 * tokens, q_item_rows) -- the output of a batched GEMV whose items are
 * q_item_rows-row slices of the q projection.
 */
int glq_qk_norm_rope(const void* q, const void* k, const void* v, int64_t tokens,
                     int64_t q_heads, int64_t kv_heads, int64_t head_dim, int64_t q_stride,
                     int64_t q_item_rows, int64_t kv_stride, const void* q_norm_w,
                     const void* k_norm_w, float eps,
                     const void* cos, const void* sin, int64_t cs_stride, void* q_out,
                     void* k_cache, void* v_cache, int64_t max_len, const int64_t* pos,
                     int32_t* len_out, void* stream);

/*
 * Workspace bytes of glq_decode_attention (per-split partial results, then
 * one arrival counter per (token, KV head)); -1 for invalid sizes.
 */
int64_t glq_decode_attention_workspace_bytes(int64_t tokens, int64_t q_heads,
                                             int64_t kv_heads, int64_t max_len);

/*
 * Single-query attention of one decode token per row over cache positions
 * [0, L), L = *len clamped to [1, max_len] (device int32, written by
 * glq_qk_norm_rope): for q head h, KV head h / (q_heads / kv_heads) (at most
 * 8 q heads per KV head),
 *   out[t][h*128 + d] = fp16(sum_p softmax_p(scale * q.k_p) v_p[d])
 * with fp32 scores, softmax and sums, split over 128-position blocks whose
 * partial results the last-arriving block merges.  q (tokens, q_heads, 128);
 * caches as in glq_qk_norm_rope; out (tokens, q_heads * 128).  workspace:
 * glq_decode_attention_workspace_bytes, 256-byte aligned; its counters must
 * be zero before the first call (each call leaves them zero), and calls that
 * share a workspace must not overlap.  When advance != NULL, *advance (device
 * int64, the cache's fill counter) is incremented by one.
 */
int glq_decode_attention(const void* q, const void* k_cache, const void* v_cache,
                         int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                         int64_t max_len, const int32_t* len, float scale, int64_t* advance,
                         void* out, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * glq_decode_attention, and in the same launch the low-rank factor of the
 * projection that reads its output (the o projection) as fp32 partials, one
 * per KV group g (the rows of its q heads):
 *   parts[g][t][j] = sum over k in group g's rows of out[t][k] U[k][j]
 * ((kv_heads, tokens, rpad), rpad = rank rounded up to 32), which
 * glq_gemv_lora_parts sums in group order as its a.  U (q_heads * 128,
 * rank) fp16, 16-byte aligned, rank a multiple of 8 (<= 1024).  Each
 * (token, KV group) block that merges the splits forms its group's partial
 * (its U rows' loads issued behind the merge's).  No reference kernel: the
 * reference forms x U inside GLoRCQLinear.forward
 * (inference/quantized_linear.py:338-345).  workspace as glq_decode_attention.
 */
int glq_decode_attention_xu(const void* q, const void* k_cache, const void* v_cache,
                            int64_t tokens, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                            int64_t max_len, const int32_t* len, float scale, int64_t* advance,
                            void* out, const void* U, int64_t rank, float* parts,
                            void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GLORCQ_HIP_H */
