/*
 * flash_mlm_hip.h -- C ABI of the MI355X (gfx950) implementation of the
 * flash-mlm fused MLM attention path.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, element
 * counts and strides (in elements, not bytes), launches asynchronously on the
 * HIP stream passed as `void* stream` (NULL = the null stream), allocates no
 * memory, and returns 0 on success, a positive hipError_t on a HIP launch
 * error, or a negative FMLM_E* code when an argument fails the library's own
 * memory-safety checks.  All shape/semantic validation that produces the
 * reference's ValueError messages stays in the host layer above this ABI.
 *
 * Reference interfaces replaced (paths relative to the flash-mlm repository):
 *   fmlm_pack_metadata  <- build_pack_metadata + _build_query_tile_map_from_cu_seqlens
 *                          src/flash_mlm/host/host_utils.py:27-71, 74-107
 *   fmlm_pack           <- _pack_flatten_for_kernel_into / pack_and_pad_main_tensors_for_mlm_compressed
 *                          / pack_for_kernel / pad_packed_main_tensors_for_mlm_compressed
 *                          src/flash_mlm/host/host_utils.py:266-289, 397-420, 423-491, 494-584
 *                          and the dense MLA prefill copy k[:,0].contiguous(),
 *                          src/flash_mlm/host/host.py:206-213
 *   fmlm_unpack         <- unpack_from_kernel, src/flash_mlm/host/host_utils.py:587-615
 *   fmlm_attn_fwd       <- _mlm_compressed_kernel[grid](...) launch, src/flash_mlm/host/host.py:471-521
 *                          and _mlm_main_kernel[grid](...) launch, src/flash_mlm/host/host.py:164-204
 *                          (device bodies src/flash_mlm/mlm_kernel_impl.py:10-62, 65-216, 219-390)
 */
#ifndef FLASH_MLM_HIP_H
#define FLASH_MLM_HIP_H

#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define FMLM_API __attribute__((visibility("default")))
#else
#define FMLM_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FMLM_ABI_VERSION 5

/* element types */
enum {
  FMLM_DTYPE_BF16 = 0,
  FMLM_DTYPE_F16 = 1,
  FMLM_DTYPE_F32 = 2
};

/* attention flags (constexpr switches of _mlm_compressed_kernel_impl, mlm_kernel_impl.py:236-238) */
enum {
  FMLM_FLAG_MLA = 1,        /* V is K (one shared latent head for main and context) */
  FMLM_FLAG_PREFILL = 2,    /* skip the cached-context segment */
  FMLM_FLAG_CAUSAL_SEQ = 4  /* sequence b attends to main tokens [0, cu_q[b+1]) */
};

/* row layouts of a [*, D] tensor addressed by (sequence b, head h, position p) */
enum {
  FMLM_LAYOUT_PADDED = 0, /* row = b*sb + h*sh + p*sn                                  */
  FMLM_LAYOUT_PACKED = 1  /* row = h*sh + (cu_q[b] + p)*sn   (sb ignored)               */
};

/* negative return codes */
enum {
  FMLM_E_ARG = -1,        /* null pointer / negative size / unsupported combination     */
  FMLM_E_DTYPE = -2,      /* unsupported dtype for this entry point                     */
  FMLM_E_HEAD_DIM = -3,   /* unsupported head dimension                                 */
  FMLM_E_ALIGN = -4,      /* pointer or stride not aligned to the element size          */
  FMLM_E_WORKSPACE = -5   /* workspace missing or smaller than fmlm_attn_workspace_bytes */
};

/* ---------------------------------------------------------------------------
 * Library information.
 * ------------------------------------------------------------------------- */
FMLM_API int fmlm_abi_version(void);
/* sizeof(fmlm_attn_params) / sizeof(fmlm_pack_tensor) as compiled, so FFI
 * mirrors can assert their struct layout. */
FMLM_API int fmlm_attn_params_size(void);
FMLM_API int fmlm_pack_tensor_size(void);

/* ---------------------------------------------------------------------------
 * Pack metadata (host_utils.py:27-107).
 *
 * lengths:       [B] int32 (lengths_is_i64 = 0) or int64 (= 1), device.
 * Outputs (device):
 *   lengths_i32   [B]            lengths as int32
 *   aux           [2*B + 6] int32:
 *                   aux[0 .. B]        cu_seqlens  = [0, cumsum(lengths)]
 *                   aux[B+1 .. B+4]    {total_tokens, n_tiles, n_bad_lengths, 0}
 *                   aux[B+5 .. 2B+5]   exclusive tile prefix (internal)
 *   token_indices [B*N] int64    first total_tokens entries = b*N + t, t < L_b, in (b, t) order
 *   batch_ids     [B*ceil(N/block_n)] int32  tile -> sequence, first n_tiles entries valid
 *   tile_starts   [B*ceil(N/block_n)] int32  tile -> packed start cu[b] + j*block_n
 * When any length lies outside [0, N] (n_bad_lengths > 0) only lengths_i32 and
 * aux are written; the caller raises.
 * ------------------------------------------------------------------------- */
FMLM_API int fmlm_pack_metadata(const void* lengths, int32_t lengths_is_i64, int32_t B, int32_t N,
                       int32_t block_n, int32_t* lengths_i32, int32_t* aux,
                       int64_t* token_indices, int32_t* batch_ids, int32_t* tile_starts,
                       void* stream);

/* ---------------------------------------------------------------------------
 * Query tile map from cu_seqlens (host_utils.py:74-107): for every sequence b and
 * j < ceil((cu[b+1]-cu[b]) / block_n), in (b, j) order, batch_ids = b and
 * tile_starts = cu[b] + j*block_n.  At most `capacity` tiles are written;
 * *count (device int32) receives the full tile count.
 * ------------------------------------------------------------------------- */
FMLM_API int fmlm_tile_map(const int32_t* cu_seqlens, int32_t B, int32_t block_n, int32_t capacity,
                           int32_t* batch_ids, int32_t* tile_starts, int32_t* count, void* stream);

/* ---------------------------------------------------------------------------
 * Pack: padded rows (b, h, p < L_b) -> head-major packed rows h*T_pad + cu[b] + p,
 * rows h*T_pad + [T, T_pad) zeroed (host_utils.py:397-420).  Up to 3 tensors
 * per launch (q, k, v).  cu_seqlens == NULL means every sequence has N tokens
 * (then T must equal B*N), which is the dense-prefill copy k[:, 0] -> [B*N, D].
 * Pack and unpack move bytes only: elem_bytes is the element size (1, 2, 4 or 8).
 * ------------------------------------------------------------------------- */
typedef struct fmlm_pack_tensor {
  const void* src; /* source base; element (b, h, p, d) at b*s_sb + h*s_sh + p*s_sn + d */
  int64_t s_sb, s_sh, s_sn;
  void* dst;       /* [heads * T_pad, D] contiguous */
  int32_t heads;   /* heads packed from this tensor (MLA k: 1) */
  int32_t reserved;
} fmlm_pack_tensor;

FMLM_API int fmlm_pack(const fmlm_pack_tensor* tensors, int32_t n_tensors, int32_t elem_bytes, int32_t B,
              int32_t N, int32_t D, const int32_t* cu_seqlens, int32_t T, int32_t T_pad,
              void* stream);

/* ---------------------------------------------------------------------------
 * Unpack: packed rows h*p_sh/D + cu[b] + p -> dst [B, H, N, D] contiguous with
 * zeros where p >= L_b (host_utils.py:587-615).  p_sh = elements between heads
 * of the packed tensor (T*D for [H*T, D]).
 * ------------------------------------------------------------------------- */
FMLM_API int fmlm_unpack(int32_t elem_bytes, const void* packed, int64_t p_sh, void* dst, int32_t B, int32_t H,
                int32_t N, int32_t D, const int32_t* cu_seqlens, void* stream);

/* ---------------------------------------------------------------------------
 * Segment copy, the kernel of a true KV append (InferenceCache.append_kv_cache): for
 * head h < H and segment c < C, rows [src_cu[c], src_cu[c+1]) of src (row h*src_sh/D +
 * i) go to rows [dst_start[c], dst_start[c] + len) of dst (row h*dst_sh/D + i); rows are
 * D elements of elem_bytes.  Offsets are clamped to src_rows / dst_rows rows per head.
 * src == NULL writes zero rows instead (the same segments of dst; src_rows still bounds
 * the offsets src_cu).
 * No counterpart in the reference, which replaces a layer's context on prefill and lists
 * appends with paged KV on its roadmap (README.md:34-41).
 * ------------------------------------------------------------------------- */
FMLM_API int fmlm_copy_segments(int32_t elem_bytes, const void* src, int64_t src_sh, int32_t src_rows,
                                const int32_t* src_cu, void* dst, int64_t dst_sh, int32_t dst_rows,
                                const int32_t* dst_start, int32_t C, int32_t H, int32_t D, void* stream);

/* ---------------------------------------------------------------------------
 * KV append in one launch (InferenceCache.append_kv_cache): for up to 2 tensors (K, V),
 * heads h < H and batches c < C, the merged head-major entry out [H*(t_old+t_new), D]
 * holds, at rows h*(t_old+t_new) + [o_c, o_{c+1}) with o = cu_old + cu_new, the old rows
 * [cu_old[c], cu_old[c+1]) of head h of `old` ([H*t_old, D]) followed by the new rows
 * [cu_new[c], cu_new[c+1]) of head h of `add` ([H*t_new, D]); rows [o_C, t_old+t_new) of
 * every head are zero.  cu_out (C+1 int32, may be NULL) receives o.  Offsets are clamped
 * to the buffers' rows.  No counterpart in the reference, which replaces a layer's
 * context on prefill and lists appends with paged KV on its roadmap (README.md:34-41).
 * ------------------------------------------------------------------------- */
typedef struct fmlm_append_tensor {
  const void* old; /* [H * t_old, D] contiguous */
  const void* add; /* [H * t_new, D] contiguous */
  void* out;       /* [H * (t_old + t_new), D] contiguous */
} fmlm_append_tensor;

FMLM_API int fmlm_kv_append(const fmlm_append_tensor* tensors, int32_t n_tensors, int32_t elem_bytes, int32_t H,
                            int32_t D, int32_t C, int32_t t_old, int32_t t_new, const int32_t* cu_old,
                            const int32_t* cu_new, int32_t* cu_out, void* stream);

/* ---------------------------------------------------------------------------
 * Fused MLM attention forward, dense and packed (mlm_kernel_impl.py:65-216, 219-390).
 *
 * For every sequence b < B, head h < H and query position p < L_b
 * (L_b = cu_seqlens_q[b+1]-cu_seqlens_q[b], or N when cu_seqlens_q == NULL):
 *   keys = [context of b] ++ [main keys of b]
 *   context (skipped with FMLM_FLAG_PREFILL): rows cb*c_sb + h*c_sh + (c0 + j)*c_sn,
 *       j < c1 - c0, where cb = ctx_index[b] clamped to [0, ctx_batch) when ctx_index
 *       is set, else (ctx_batch > 1 ? b : 0), and
 *       (c0, c1) = (cu_seqlens_kv[cb], cu_seqlens_kv[cb+1]) clamped to [0, ctx_rows], or
 *       (0, ctx_len) when cu_seqlens_kv == NULL
 *   main: packed token indices [cu_q[b], cu_q[b+1]), or [0, cu_q[b+1]) with
 *       FMLM_FLAG_CAUSAL_SEQ, addressed through kv_layout
 *   o[b,h,p] = softmax(scale * q[b,h,p] . keys^T) @ values
 * V is K when FMLM_FLAG_MLA is set (v/v_ctx ignored).  bf16/f16 use MFMA with
 * fp32 accumulation and the probabilities rounded to the input type before
 * P.V, as the reference does (mlm_kernel_impl.py:56-58); f32 runs in fp32.
 * L_b is clamped to N (when N > 0) and to total_q - cu_seqlens_q[b].  Rows p >= L_b of
 * the output are not written.
 * ------------------------------------------------------------------------- */
#define FMLM_PAGE_ROWS 64  /* rows per page of a paged context (the kernels' key tile) */

typedef struct fmlm_attn_params {
  int32_t dtype;           /* FMLM_DTYPE_* of q, k, v, contexts and o                */
  int32_t flags;           /* FMLM_FLAG_*                                            */
  int32_t B, H, D;         /* sequences, heads, head dim                             */
  int32_t N;               /* padded per-sequence length                             */
  int32_t total_q;         /* upper bound of sum(L_b) (T or T_pad); B*N when dense   */
  int32_t ctx_len;         /* context length when cu_seqlens_kv == NULL              */
  int32_t ctx_batch;       /* context batch count; 1 => every b uses context batch 0 */
  int32_t ctx_rows;        /* rows per head of a packed context; (c0, c1) are clamped to it */
  int32_t q_layout, o_layout, kv_layout; /* FMLM_LAYOUT_*                          */
  float scale;             /* softmax scale applied to q.k                           */
  const int32_t* cu_seqlens_q;  /* [B+1] or NULL (all sequences have N tokens)      */
  const int32_t* cu_seqlens_kv; /* [ctx_batch+1] or NULL (uniform ctx_len)          */
  const void* q; int64_t q_sb, q_sh, q_sn;
  void* o;       int64_t o_sb, o_sh, o_sn;
  const void* k; int64_t k_sb, k_sh, k_sn;
  const void* v; int64_t v_sb, v_sh, v_sn;
  const void* k_ctx; const void* v_ctx; int64_t c_sb, c_sh, c_sn;
  void* workspace;         /* device scratch for the work schedule                  */
  int64_t workspace_bytes;
  const void* schedule;    /* NULL, or a schedule built by fmlm_attn_schedule for the same
                              cu_seqlens_q contents, B, H, total_q, dtype, D, flags and
                              kv_layout: then fmlm_attn_fwd launches the attention
                              kernel (plus the split merge) only.  Context lengths may
                              differ; they only steer where key ranges are split.  The
                              buffer also holds split partial results: launches that may
                              overlap need separate schedule buffers                  */
  const int32_t* ctx_index;  /* [B] context batch of each sequence, or NULL (see above):
                                index-mapped context batching.  No counterpart in the
                                reference, whose roadmap lists it ("variable context
                                batch sizes", README.md:34-36)                         */
  /* Paged context (NULL block table: contiguous context as above).  Context batch cb has
   * cu_seqlens_kv[cb+1] - cu_seqlens_kv[cb] rows (or ctx_len); its row j lives in page
   * ctx_block_table[cb * ctx_pages_per_batch + j / FMLM_PAGE_ROWS], row j % FMLM_PAGE_ROWS:
   * element page * ctx_page_stride + h * c_sh + (j % FMLM_PAGE_ROWS) * c_sn of k_ctx /
   * v_ctx.  ctx_rows is then the number of pages in the pool (page ids are clamped to it).
   * bf16/f16 with linear main keys only.  No counterpart in the reference, whose roadmap
   * lists paged KV (README.md:41).                                                     */
  const int32_t* ctx_block_table;
  int64_t ctx_page_stride;
  int32_t ctx_pages_per_batch;
  /* Tile configuration of the bf16/f16 attention kernel: 0 = chosen by the library from
   * the head dim and the query rows per sequence (D = 64 and 128: configuration 3 when
   * total_q <= 64 * B, i.e. sequences of at most 64 query rows on average, else 1; other
   * head dims: 1); k >= 1
   * forces compiled configuration k of the head dim (fmlm_attn_workspace_bytes returns
   * FMLM_E_ARG for a k that does not exist).  Configurations, as (query rows per
   * workgroup, waves per workgroup): D = 16, 32: 1 = (128, 4); D = 64: 1 = (128, 4),
   * 2 = (256, 8), 3 = (64, 4), 4 = (256, 8) ping-pong; D = 128: 1 = (128, 4),
   * 2 = (256, 8), 3 = (64, 4), 4 = (128, 8), 5 = (256, 8) ping-pong; D = 256:
   * 1 = (64, 4), 2 = (128, 8); MLA D = 512: 1 = (128, 8).  Ping-pong: the 8 waves run as
   * two groups half a key tile apart, so that one wave of each SIMD computes softmax
   * while the other issues MFMAs.  Replaces the reference's autotuned
   * BLOCK_M / BLOCK_N / num_warps (mlm_kernel.py:57-166).  Ignored by f32 inputs.       */
  int32_t tile_config;
  /* Row statistics for the backward: NULL, or H * total_q floats that fmlm_attn_fwd fills
   * with each real query row's log2-sum-exp, row p of sequence b and head h at
   * h * total_q + q0_b + p (q0_b = cu_seqlens_q[b], or b * N without cu_seqlens_q):
   * log2(sum over its keys of 2^z), z = scale * log2(e) * q.k as the forward kernel
   * computes it (fp32 accumulation); +inf for a row without keys.
   * fmlm_attn_bwd given the same block reads it instead of recomputing it.  No
   * counterpart in the reference, whose kernels return o only.                        */
  float* lse;
} fmlm_attn_params;

/* Bytes of device workspace (and of a schedule buffer) fmlm_attn_fwd needs for these
 * parameters (>= 0), or < 0 on unsupported dtype / head dim. */
FMLM_API int64_t fmlm_attn_workspace_bytes(const fmlm_attn_params* p);

/* Build the work schedule (one entry per query tile of the kernel's own tile size over
 * the real rows of every sequence) into `schedule` (fmlm_attn_workspace_bytes bytes) so
 * later fmlm_attn_fwd calls with p->schedule = schedule skip rebuilding it.  No
 * counterpart in the reference (its tile map is PackMetadata.batch_ids_q /
 * q_tile_starts_q at block_n granularity, host_utils.py:74-107). */
FMLM_API int fmlm_attn_schedule(const fmlm_attn_params* p, void* schedule, int64_t schedule_bytes,
                                void* stream);

FMLM_API int fmlm_attn_fwd(const fmlm_attn_params* p, void* stream);

/* ---------------------------------------------------------------------------
 * fmlm_attn_fwd without a workspace, for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * No counterpart in the reference.  Same parameters and results as fmlm_attn_fwd;
 * p->workspace and p->schedule are ignored.  The work schedule and the split-KV partial
 * results live in a device array owned by the library, FMLM_NOALLOC_SCRATCH_BYTES per
 * GPU, held until the process ends; the schedule is rebuilt on every call.  When the
 * split records would not fit, fewer key ranges are split (or none); a call whose
 * unsplit schedule does not fit returns FMLM_E_WORKSPACE.  Every call on a GPU shares
 * that GPU's array: calls that may overlap on one GPU (different streams, or host
 * threads) race and must be serialised by the caller.  Allocates nothing.
 * ------------------------------------------------------------------------- */
#define FMLM_NOALLOC_SCRATCH_BYTES (16 << 20)

FMLM_API int fmlm_attn_fwd_noalloc(const fmlm_attn_params* p, void* stream);

/* ---------------------------------------------------------------------------
 * Attention backward.  No counterpart in the reference, whose roadmap lists
 * backpropagation (README.md:26-28); it differentiates fmlm_attn_fwd for the same
 * parameter block p (p->o holding that call's output):
 *   dq      rows laid out like q (q_layout) with the dq strides: every real row
 *   dk, dv  main-key rows laid out like k / v (kv_layout) with the dk / dv strides: every
 *           key row some query attends to.  With FMLM_FLAG_MLA dk receives the gradient
 *           of K and of V (V is K) and dv is unused.  Keys with head stride 0 (the MLA
 *           latent) are shared by all heads, and so is their gradient row (dk_sh = 0).
 *   dk_ctx, dv_ctx  the context's gradient, laid out like k_ctx / v_ctx (c_sb, c_sh,
 *           c_sn), or NULL to skip it: rows [c0, c1) of every context batch.  With a
 *           paged context (ctx_block_table) they are float32 buffers laid out like the
 *           pool, zeroed by the caller, that the kernel adds into atomically: a page used
 *           by several context batches receives the sum of their gradients.
 * Rows not listed are not written.  dout is laid out like o (o_layout).
 * bf16 / f16 (MFMA) and f32 (SIMT), D in {16, 32, 64, 128, 256, 512}; with
 * FMLM_FLAG_CAUSAL_SEQ the main keys must be packed (kv_layout PACKED).
 * workspace: fmlm_attn_bwd_workspace_bytes(p) bytes (per-row softmax statistics, the
 *           tile tables of the two kernels and a 64-byte record per tile).
 * ------------------------------------------------------------------------- */
typedef struct fmlm_attn_grads {
  const void* dout; int64_t do_sb, do_sh, do_sn;
  void* dq;  int64_t dq_sb, dq_sh, dq_sn;
  void* dk;  int64_t dk_sb, dk_sh, dk_sn;
  void* dv;  int64_t dv_sb, dv_sh, dv_sn;
  void* dk_ctx;
  void* dv_ctx;
  void* workspace;
  int64_t workspace_bytes;
} fmlm_attn_grads;

FMLM_API int fmlm_attn_grads_size(void);  /* sizeof(fmlm_attn_grads), for bindings */
FMLM_API int64_t fmlm_attn_bwd_workspace_bytes(const fmlm_attn_params* p);
FMLM_API int fmlm_attn_bwd(const fmlm_attn_params* p, const fmlm_attn_grads* g, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_MLM_HIP_H */
