/*
 * kernel_lab C-ABI: fused residual-add + RMSNorm and paged-KV decode attention
 * for AMD Instinct MI355X (gfx950).
 *
 * The header is plain C. It includes no HIP, PyTorch or C++ header, so any
 * FFI (ctypes, cgo, JNI, a C++ serving loop) can bind it directly. Every
 * pointer is a device pointer unless stated otherwise; every launch is
 * asynchronous on `stream` and never synchronises the host.
 *
 * Reference interface replaced: `kernel_lab::launch_rms_norm` and
 * `kernel_lab::launch_paged_decode_attention` in csrc/kernel_lab.h:17-33 of
 * Markkoby3/Kernel-lab, plus the split-KV contract of
 * kernel_lab/triton_kernels/paged_attention.py:169-264 (num_splits,
 * max_seq_len, fp32 partials).
 */
#ifndef KERNEL_LAB_H_
#define KERNEL_LAB_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same handle type as HIP's hipStream_t, declared without including HIP. */
typedef struct ihipStream_t* kl_stream_t;

/* Element types. Replaces `enum class DType` (csrc/kernel_lab.h:12). In C++
 * the type is int-based, so any int a C caller passes is a value of it and
 * reaches the library's checks, which reject values outside the list. */
typedef enum kl_dtype
#ifdef __cplusplus
    : int
#endif
{
  KL_DTYPE_F32 = 0,
  KL_DTYPE_F16 = 1,
  KL_DTYPE_BF16 = 2
} kl_dtype;

/* num_splits value asking paged decode for the device-balanced schedule. */
#define KL_SPLITS_BALANCED (-1)

/* kl_paged_decode_last_merge results. */
#define KL_MERGE_NONE 0      /* no sequence was split (or the call failed)   */
#define KL_MERGE_KERNEL 1    /* split sequences merged by a second launch    */
#define KL_MERGE_IN_KERNEL 2 /* merged by the decode kernel's last segment   */

/*
 * Status codes. The reference launchers return cudaError_t and signal
 * unsupported shapes with cudaErrorInvalidValue (csrc/paged_attention.cu:157,
 * 174, 198); here argument errors and runtime errors are told apart.
 */
typedef enum kl_status {
  KL_OK = 0,
  KL_ERR_INVALID_ARGUMENT = 1, /* bad pointer, size, dtype or stride        */
  KL_ERR_UNSUPPORTED = 2,      /* a shape this build has no kernel for      */
  KL_ERR_WORKSPACE = 3,        /* workspace missing or smaller than needed  */
  KL_ERR_HIP = 4               /* the HIP runtime reported an error         */
} kl_status;

/* Static text for a status code. */
const char* kl_status_string(int status);

/*
 * Detail of the last failed call on the calling thread (argument name,
 * HIP error text), or "" if the last call succeeded. Valid until the next
 * kernel_lab call on this thread.
 */
const char* kl_last_error(void);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int kl_version(void);

/*
 * RMSNorm over `rows` rows of length `hidden`.
 * Replaces kernel_lab::launch_rms_norm (csrc/kernel_lab.h:14-19).
 *
 *   residual == NULL:  out = rmsnorm(x) * weight
 *   residual != NULL:  residual = dtype(f32(x) + f32(residual))   (in place)
 *                      out      = rmsnorm(residual) * weight
 *
 * `out`, `residual` and `weight` are contiguous; row i of `x` starts at
 * x + i * x_row_stride elements (x_row_stride >= hidden). rows == 0 is a
 * successful no-op. Math is fp32; `out` is rounded to nearest even.
 */
int kl_rms_norm(kl_dtype dtype, void* out, const void* x, void* residual, const void* weight,
                int64_t rows, int64_t hidden, int64_t x_row_stride, float eps,
                kl_stream_t stream);

/*
 * Split planning for paged decode. Pure host arithmetic: it reads no device
 * memory (in particular not seq_lens), so it never synchronises.
 * Follows choose_num_splits and the split normalisation of
 * kernel_lab/triton_kernels/paged_attention.py:169-173,205-211, with the
 * workgroup target sized for the device's compute units.
 *
 *   max_pages        block-table columns any sequence may use
 *                    (= cdiv(max_seq_len, page_size) when that is known)
 *   num_splits       requested KV splits; 0 lets the planner choose;
 *                    KL_SPLITS_BALANCED asks for the balanced schedule at any
 *                    batch size (fp16/bf16 MFMA shapes; elsewhere it acts as 0)
 *   cu_count         compute units to plan for; 0 queries the current device
 *   out_num_splits   (host pointer) uniform splits the launch will use, or 0
 *                    when it balances pages across sequences on the device
 *                    (chosen for fp16/bf16 batches of two or more sequences
 *                    when there are fewer (sequence, KV head) units than
 *                    compute units, and for full batches while the balanced
 *                    workspace stays within 16 MiB: one workgroup per unit,
 *                    which on an even batch is one uniform split's cut,
 *                    detected on the device; full batches of more than 8
 *                    query heads per KV head take it only when the table
 *                    spans >= 256 pages; a single sequence takes uniform
 *                    splits of >= 8 pages)
 *   out_workspace    (host pointer) bytes of device workspace the launch needs
 *                    (0 when the launch needs none)
 */
int kl_paged_decode_plan(kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads,
                         int head_dim, int page_size, int max_pages, int num_splits,
                         int cu_count, int* out_num_splits, size_t* out_workspace);

/*
 * Single-token decode attention over a paged KV cache (NHD layout).
 * Replaces kernel_lab::launch_paged_decode_attention (csrc/kernel_lab.h:21-33)
 * and the split-KV wrapper of kernel_lab/triton_kernels/paged_attention.py:176-264.
 *
 *   q, out        [batch, num_q_heads, head_dim]                    contiguous
 *   k/v_cache     [num_pages, page_size, num_kv_heads, head_dim]    contiguous
 *   block_table   [batch, block_table_stride] int32 page ids
 *   seq_lens      [batch] int32, each in [1, max_pages * page_size]
 *
 * Sequence b attends over its first seq_lens[b] cached tokens, following
 * block_table[b, 0 .. cdiv(seq_lens[b], page_size)). Entries past that and
 * pages not named there are never read. num_q_heads must be a multiple of
 * num_kv_heads (grouped-query attention). `scale` multiplies q.k.
 * num_splits == 0 lets the planner choose; KL_SPLITS_BALANCED (-1) cuts the
 * pages of all sequences into equal per-workgroup ranges on the device, which
 * suits batches of very uneven lengths (on a batch of at most 256 sequences
 * whose page counts differ, each (sequence, KV head) unit also counts a few
 * pages for the segment start it costs, so ranges that start a unit are
 * shorter). Block tables long enough that 64 sequences' units would pass
 * 2^31 pages take uniform splits instead. The workspace must hold at least
 * the bytes kl_paged_decode_plan reports for the same arguments; it may be
 * NULL when that is 0. batch == 0 is a successful no-op.
 *
 * Split sequences are merged inside the decode kernel where the path allows
 * it (fp16/bf16, at most 8 query heads per KV head and head group, and a
 * sequence cut into few enough segments that one workgroup's merge stays
 * short; otherwise a separate merge launch runs). The library keeps
 * per-device arrival counters (8 MiB) in regions that calls able to overlap
 * never share: an eager call uses its stream's region (64 streams per
 * device), a call recorded under graph capture a region of its own capture
 * sequence and stream (192 per device, never reused), so graphs may replay
 * concurrently on any streams. hipStreamPerThread, and streams or captures
 * beyond those counts (reported once on stderr), use the merge launch;
 * results are bit-identical either way. KL_DECODE_FUSED_MERGE=0 in the
 * environment forces the merge launch (see kl_paged_decode_reload_options).
 */
int kl_paged_decode_attention(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                              const void* v_cache, const int32_t* block_table,
                              const int32_t* seq_lens, int batch, int num_q_heads,
                              int num_kv_heads, int head_dim, int page_size,
                              int64_t block_table_stride, int max_pages, float scale,
                              int num_splits, void* workspace, size_t workspace_bytes,
                              kl_stream_t stream);

/*
 * How the last paged-decode call on the calling thread (any of the
 * kl_paged_decode_attention entry points) combined split sequences: one of
 * KL_MERGE_NONE, KL_MERGE_KERNEL, KL_MERGE_IN_KERNEL. A diagnostic for
 * performance work and tests; no counterpart in the reference, whose
 * launchers do not split sequences.
 */
int kl_paged_decode_last_merge(void);

/*
 * Re-reads the decode switches from the environment. The library reads them
 * once per process, at its first decode call; tests and A/B measurements
 * that change them afterwards call this. No counterpart in the reference.
 *   KL_DECODE_FORCE_VALU=1        fp16/bf16 decode on the VALU kernel
 *   KL_DECODE_PAIRED=0            no two-KV-head workgroups
 *   KL_DECODE_BALANCE_ALWAYS=1|0  full batches always / never balanced
 *   KL_DECODE_FUSED_MERGE=0       split sequences merged by a second launch
 * KL_DECODE_PAIRED and KL_DECODE_FUSED_MERGE leave the output bits unchanged
 * (except where a full batch's default schedule depends on the fused merge
 * being available); the other two change how the work is cut or computed,
 * so outputs agree within the decode tolerance but not bit for bit.
 * Returns KL_OK.
 */
int kl_paged_decode_reload_options(void);

/*
 * kl_paged_decode_attention without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid allocation). It has no counterpart in the reference.
 *
 * The split workspace lives in a library-owned 16 MiB device array, one per
 * device, held until the process ends; it fits every split the planner
 * chooses by itself (num_splits 0). A plan needing more (explicit split
 * counts over large batches) returns KL_ERR_WORKSPACE without launching.
 * The first call on a device looks up that device's array; the call
 * allocates nothing (no hipMalloc, no hipFree). Calls that overlap on one
 * device share the array and race: run them on one stream, or use
 * kl_paged_decode_attention with a workspace per stream. Other arguments,
 * results and status codes are those of kl_paged_decode_attention.
 */
int kl_paged_decode_attention_noalloc(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                      const void* v_cache, const int32_t* block_table,
                                      const int32_t* seq_lens, int batch, int num_q_heads,
                                      int num_kv_heads, int head_dim, int page_size,
                                      int64_t block_table_stride, int max_pages, float scale,
                                      int num_splits, kl_stream_t stream);

/*
 * Paged decode over an FP8 KV cache: k_cache / v_cache hold OCP FP8 E4M3
 * codes ("e4m3fn": bias 7, no infinities, 0x7f / 0xff are NaN), one byte per
 * element, in the same [num_pages, page_size, num_kv_heads, head_dim] layout;
 * head h's values are k_scale[h] * decode(k) and v_scale[h] * decode(v)
 * (k_scale, v_scale: [num_kv_heads] fp32 device arrays). q and out are fp16
 * or bf16 (`dtype`); the cache values are decoded exactly to that type, so
 * the arithmetic is that of kl_paged_decode_attention.
 *
 * Reference counterpart: none in the shipped kernels; the original project
 * names an FP8 KV cache as planned work (README.md:98). Arguments, workspace
 * (size it with kl_paged_decode_plan for the same dtype and shape) and status
 * codes are those of kl_paged_decode_attention; head_dim must be 64, 128 or
 * 256 and page_size a multiple of 16 (KL_ERR_UNSUPPORTED otherwise).
 */
int kl_paged_decode_attention_fp8(kl_dtype dtype, void* out, const void* q,
                                  const void* k_cache, const void* v_cache,
                                  const float* k_scale, const float* v_scale,
                                  const int32_t* block_table, const int32_t* seq_lens,
                                  int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                  int page_size, int64_t block_table_stride, int max_pages,
                                  float scale, int num_splits, void* workspace,
                                  size_t workspace_bytes, kl_stream_t stream);

/*
 * Cascade (shared-prefix) decode: sequence b attends over the prefix_len[0]
 * tokens of the shared prefix (pages prefix_block_table[0 .. prefix_pages))
 * followed by its own seq_lens[b] tokens (pages block_table[b, ...]), all in
 * the same k_cache / v_cache pools. The result is the attention over the
 * concatenated tokens; a sequence may have no own tokens (seq_lens[b] == 0),
 * and prefix_pages == 0 makes it plain decode.
 *
 * Reference counterpart: none in the shipped kernels; the original project's
 * design notes name cascade/shared-prefix attention among the decode
 * features beyond its kernels (docs/design.md:96-100). The prefix's K/V is
 * streamed once per 32 query heads of the folded batch instead of once per
 * sequence.
 *
 *   prefix_len   device pointer to one int32 (no host sync)
 *   workspace    at least kl_cascade_decode_plan's bytes, 16-byte aligned
 *
 * fp16 / bf16, head_dim 32..256, page_size a multiple of 16; other arguments
 * and status codes as kl_paged_decode_attention.
 */
int kl_cascade_decode_plan(kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads,
                           int head_dim, int page_size, int prefix_pages, int max_pages,
                           int cu_count, size_t* out_workspace);

int kl_cascade_decode_attention(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                const void* v_cache, const int32_t* prefix_block_table,
                                const int32_t* prefix_len, int prefix_pages,
                                const int32_t* block_table, const int32_t* seq_lens, int batch,
                                int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                int64_t block_table_stride, int max_pages, float scale,
                                void* workspace, size_t workspace_bytes, kl_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* KERNEL_LAB_H_ */
