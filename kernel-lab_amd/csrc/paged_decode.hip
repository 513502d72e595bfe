// Paged-KV decode attention for gfx950: split-KV flash-decoding with GQA
// packing and an exact base-2 log-sum-exp merge.
//
// Behavioural spec: kernel_lab/triton_kernels/paged_attention.py:37-264
// (split kernel, merge kernel, split planner) and kernel_lab/reference.py:33-68
// (the math). Drop-in boundary: csrc/paged_attention.cu:180-199 and
// csrc/kernel_lab.h:21-33.
//
// Work unit: (sequence b, KV head, head group) and a range of its pages. Two
// schedules cut the units into workgroup segments:
//   uniform splits   a split owns `pages_per_split` pages of every unit (the
//                    original project's rule); one workgroup per (unit, split);
//   balanced         the pages of all units are laid end to end and cut into
//                    equal per-workgroup ranges on the device from seq_lens, so
//                    a long sequence among short ones is spread over many
//                    workgroups (chosen when units do not fill the device, or
//                    on request).
// A segment runs on four waves; its 16-token blocks go round-robin to the
// waves, each wave keeps its own running max / normaliser / output, and the
// waves merge through LDS at the end. Uniform splits on a device they fill
// twice over run two segments per 8-wave workgroup, KV heads 2j and 2j+1 of
// one sequence side by side (adjacent bytes of every token row). A segment that covers its whole unit
// writes the final output; otherwise it writes an fp32 partial output and its
// log2-sum-exp, and a merge kernel combines the partials of each (sequence,
// query head).
//
// MFMA path (fp16 / bf16, page_size % 16 == 0, head_dim in {32,64,128,256}):
//   S  = K . Q^T    v_mfma_f32_16x16x32_{f16,bf16}: rows = 16 tokens of a
//                   block, columns = up to 16 query heads of the GQA group.
//                   K is loaded row-coalesced (16 lanes read one token's head
//                   dims), restaged through a per-wave LDS tile and read back
//                   as the A operand (lane = token, 8 consecutive head dims).
//   O^T += V^T P^T  v_mfma_f32_16x16x32_{f16,bf16}: the score tile's output
//                   layout (lane = head, 4 consecutive tokens) is the B operand
//                   layout, so P never leaves registers; P goes in as a 16-bit
//                   high part and low part (k = the block's tokens twice), so
//                   the weights keep ~17-21 bits. V is loaded the same
//                   row-coalesced way, staged in LDS and read back transposed
//                   (ds_read_b64_tr_b16) as the A operand.
// Every K/V element is read from HBM once per unit and used by the whole GQA
// group. Tokens past seq_len inside the last page are excluded by selects
// (scores to -inf, V rows to zero), never by multiplying by zero, so NaN or
// garbage there cannot leak; pages past cdiv(seq_len, page_size) and pages not
// named by the block table are never read.
//
// VALU path (fp32, and shapes the MFMA path does not take): lanes own 16-byte
// slices of a token's head dims; dot products reduce across the lanes of a
// token; each lane keeps an online softmax per query head and lanes merge by
// the log-sum-exp rule at the end.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <atomic>
#include <mutex>
#include <vector>
#include <type_traits>

#include "hip_common.h"
#include "kl_internal.h"

namespace kl {
namespace {

// Tuning constants, each the measured best on MI355X.
constexpr int kWaves = 4;  // waves per workgroup (a KV-head pair's workgroup has two sets)
constexpr int kThreads = kWaves * 64;
constexpr int kBlock = 16;     // tokens per MFMA block
constexpr int kMaxPlannedSplits = 64;
constexpr int kMinPagesPerSplit = 16;      // fewest pages a planned uniform split takes
constexpr int kMinPagesPerSingleSplit = 8;  // the same for a batch of one sequence
constexpr int kMinPagesPerBalancedWg = 8;  // fewest pages a balanced-schedule workgroup takes
// The balanced cut's charge for a segment start, in K/V bytes of one
// workgroup's stream (balanced_charge), and its cap in pages.
constexpr int64_t kSegmentStartBytes = 128 * 1024;
constexpr int kMaxSegmentCharge = 64;
constexpr int kFusedMaxSegments = 8;       // most segments of a balanced unit merged in the kernel
constexpr int kMinSegmentPages = 32;       // ... while its segments are shorter than this (make_plan)
// Cache policy of the K/V loads: streamed once, so non-temporal. Measured on
// 32/8/128 fp16 B=64 ctx 4096: nt 173 us, nt with sc0 and/or sc1 172.5-173.7,
// no policy bits 221.
constexpr int kKvPolicy = kCachePolicyNT;
// A batch with fewer units than 2 x CUs runs the balanced schedule in KV-head
// pairs when every workgroup half streams at least kPairMinPages pages and no
// pair unit is cut into more than kPairMaxSegments segments. Measured on
// MI355X (fp16/bf16, events): 64/8/128 B=8 ctx 32768 185 -> 176 us, ctx
// 131072 704 -> 667 us, 32/8/128 B=8 ctx 32768 183 -> 175 us; shorter
// segments lose to the 8-wave start (B=8 ctx 4096 +1.9 us) and many-way
// splits to the merge (64/8/128 B=1 ctx 32768, 64 segments: +6 us).
constexpr int kPairMinPages = 128;
constexpr int kPairMaxSegments = 16;
// Full batches take the balanced schedule by default as long as its
// workspace stays within kAutoBalanceMaxWorkspace (the no-allocation entry
// point's array); those whose split units would need the separate merge
// launch only from this many block-table columns on (see make_plan).
constexpr int kBalanceMinPages = 256;
constexpr size_t kAutoBalanceMaxWorkspace = size_t{16} << 20;
constexpr float kLog2e = 1.4426950408889634f;
// How far (log2 units) a score may pass the decode's running reference max
// before the outputs are rescaled to a new one: weights stay below 2^8.
constexpr float kRescaleSlack = 8.0f;

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const int32_t* block_table;
  const int32_t* seq_lens;
  const float* k_scale;  // [num_kv_heads] dequantisation scales of an FP8 cache; null otherwise
  const float* v_scale;
  float* o_part;    // [batch, num_q_heads, num_splits, head_dim]
  float* lse_part;  // [batch, num_q_heads, num_splits], log2 domain
  int64_t bt_stride;
  int64_t page_stride;  // elements between pages: page_size * num_kv_heads * head_dim
  int token_stride;     // elements between tokens of a page: num_kv_heads * head_dim
  int batch;
  int num_q_heads;
  int num_kv_heads;
  int group;            // num_q_heads / num_kv_heads
  int page_size;
  // Blocks per page (page_size / 16) as a multiplier and shift: for
  // 0 <= n < 2^31, n / bpp == (n * bpp_magic) >> bpp_shift (set_page_size).
  // The block -> page division runs for every block of the MFMA loops, where a
  // division by a run-time integer costs ~20 scalar instructions.
  uint32_t bpp_magic;
  int bpp_shift;
  int max_pages;
  int num_splits;
  int pages_per_split;
  int head_groups;      // workgroups per (sequence, KV head, split) along the group
  int heads_per_wg;     // query heads one workgroup handles
  int grid;             // workgroups of the balanced decode kernel (0: uniform splits)
  // Balanced kernel: 1 when the grid is one workgroup per list unit and the
  // batch has at most 64 * kScanChunks sequences, else 0 (see
  // decode_mfma_balanced_kernel's even-batch start).
  int even_start;
  // Balanced kernel: list positions the cut charges for starting a unit's
  // segment, on top of its pages (balanced_charge); the kernel applies it to
  // uneven batches of at most 64 * kScanChunks sequences only.
  int seg_charge;
  float scale_log2;     // scale * log2(e)
  // Query-row mapping. Local head hl of KV head kvh in sequence b reads q row
  // (b + hl / q_fold) * q_heads + kvh * q_fold + hl % q_fold, and the output
  // has q's layout. Plain decode: q_fold = group, q_heads = num_q_heads (the
  // identity). The shared-prefix pass of cascade decode folds every
  // sequence's group into one: batch 1, group = B * G, q_fold = G.
  int q_fold;
  int q_heads;
  int force_partial;    // write fp32 partials (o, lse) even with one split
  int paired;           // host only: uniform splits run two units per workgroup (decode_mfma_paired_kernel)
  // Fused merge: this call's arrival counters, one per unit, zero on entry
  // and left zero (null: a merge kernel combines the partials).
  uint32_t* arrivals;
};

// Block index -> page index (n >= 0, wave-uniform or per lane).
__device__ __forceinline__ int block_page(const DecodeArgs& a, int n) {
  return static_cast<int>((static_cast<uint64_t>(static_cast<uint32_t>(n)) * a.bpp_magic) >> a.bpp_shift);
}

struct Unit {
  int b, kvh, hg, split;
  int seq_len;          // clamped to max_pages * page_size
  int page_begin, page_end;
};

// The sequence length and this split's page range of a unit whose b and
// split are set.
__device__ __forceinline__ void unit_pages(const DecodeArgs& a, Unit& u) {
  const int raw = as_constant(a.seq_lens)[u.b];
  const int64_t cap = static_cast<int64_t>(a.max_pages) * a.page_size;
  u.seq_len = static_cast<int>(raw < cap ? raw : cap);
  const int num_pages = u.seq_len > 0 ? (u.seq_len + a.page_size - 1) / a.page_size : 0;
  u.page_begin = u.split * a.pages_per_split;
  u.page_end = min(u.page_begin + a.pages_per_split, num_pages);
}

// The unit of a uniform-split workgroup: b, kvh, hg and split from the
// workgroup index (no memory access), then its length and page range.
__device__ __forceinline__ Unit decode_unit_ids(const DecodeArgs& a) {
  Unit u;
  int idx = static_cast<int>(blockIdx.x);
  u.split = idx % a.num_splits;
  idx /= a.num_splits;
  u.hg = idx % a.head_groups;
  idx /= a.head_groups;
  u.kvh = idx % a.num_kv_heads;
  u.b = idx / a.num_kv_heads;
  return u;
}

__device__ __forceinline__ Unit decode_unit(const DecodeArgs& a) {
  Unit u = decode_unit_ids(a);
  unit_pages(a, u);
  return u;
}

// Paired workgroups (num_kv_heads even): workgroup i holds the units of KV
// heads 2j and 2j+1 of one (sequence, head group, split), half `half`
// taking KV head 2j + half. The digits of i are split (fastest), head
// group, KV-head pair j, sequence.
__device__ __forceinline__ Unit decode_unit_paired_ids(const DecodeArgs& a, int half) {
  Unit u;
  int idx = static_cast<int>(blockIdx.x);
  u.split = idx % a.num_splits;
  idx /= a.num_splits;
  u.hg = idx % a.head_groups;
  idx /= a.head_groups;
  const int pairs = a.num_kv_heads / 2;
  u.kvh = 2 * (idx % pairs) + half;
  u.b = idx / pairs;
  return u;
}

// Writes zeros for the heads of an empty sequence (seq_len <= 0). The math of
// kernel_lab/reference.py:58-67 gives zeros there (softmax over no tokens, then
// an empty weighted sum).
// Threads tid = 0 .. nthreads-1 of the unit's workgroup (or half) share the work.
template <typename S, typename E>
__device__ void write_zero_heads(const DecodeArgs& a, const Unit& u, int head_dim, int tid, int nthreads) {
  const int h0 = u.hg * a.heads_per_wg;
  const int nh = min(a.heads_per_wg, a.group - h0);
  S* out = static_cast<S*>(a.out);
  for (int i = tid; i < nh * head_dim; i += nthreads) {
    const int h = u.kvh * a.group + h0 + i / head_dim;
    out[(static_cast<int64_t>(u.b) * a.num_q_heads + h) * head_dim + i % head_dim] = E::from_f32(0.0f);
  }
}

// ------------------------------------------------------------ MFMA split path

// 16x16x32 products: lane l holds A[row l % 16][k in group l / 16] and
// B[k in group l / 16][col l % 16], eight k values each; element e of a lane's
// A operand meets element e of the B operand of the lane with the same k group.
template <typename E>
struct Mfma;

template <>
struct Mfma<F16> {
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
};

template <>
struct Mfma<BF16> {
  static __device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
};

// O^T += V^T (P_hi + P_lo)^T over one 16-token block in one 16x16x32 product.
// The softmax weights P are fp32; one 16-bit value keeps 8 (bf16) or 11
// (fp16) of their bits, which left outputs near zero several ulps from the
// float32 result. P is carried as a pair: P_hi = E(P) and P_lo = E(P - P_hi)
// (P - P_hi is exact in fp32), good to about 2^-17 of P in bf16 and 2^-21 in
// fp16. The k dimension holds each lane's four tokens twice: V rows against
// P_hi, then the same V rows against P_lo. `v` holds V^T[dim][tokens 4g ..
// 4g+3] (the transposing LDS read), `p_hi` / `p_lo` P[tokens 4g .. 4g+3][head].
template <typename E>
__device__ __forceinline__ f32x4 pv_split(u32x2 v, u32x2 p_hi, u32x2 p_lo, f32x4 c) {
  return Mfma<E>::mma(u32x4{v[0], v[1], v[0], v[1]}, u32x4{p_hi[0], p_hi[1], p_lo[0], p_lo[1]}, c);
}

// The low part of a packed pair of weights: E(p - f32(E(p))) for both halves.
template <typename E>
__device__ __forceinline__ uint32_t pack2_residual(float a, float b, uint32_t hi) {
  return pack2<E>(a - lo_f32<E>(hi), b - hi_f32<E>(hi));
}

// Depth of the LDS pipeline: blocks per wave in LDS at once. Measured on
// MI355X (events, same tensors): 3 and 4 stages were slower at every shape
// tried (32/8/128 fp16 B=8 ctx 4096 30.8 -> 32.9 / 32.3 us, B=1 ctx 4096
// 16.8 -> 17.6 / 19.3, ragged MQA 45.7 -> 47.7 / 50.2), as deeper register
// pipelines were: more bytes in flight per wave lower HBM throughput here.
constexpr int kDmaStages = 2;

// LDS bytes the MFMA kernel needs: the per-wave K and V staging tiles during
// the main loop, reused for the cross-wave merge afterwards (every wave's
// output tiles, 16 bytes per lane each, and its running max and normaliser).
template <int D, int NT, int W = kWaves, bool DMA = false, int NSD = kDmaStages>
struct MfmaLds {
  // Register pipeline (DMA false): one block per wave staged at a time. Row
  // strides of a staged token: K's 8 elements (16 B) of pad put the 16 rows
  // one ds_read_b128 touches on distinct 16-byte bank groups; V's 16 elements
  // of pad put the 16 rows a transposing read touches on distinct 32-byte
  // bank groups two by two.
  static constexpr int kKRow = D + 8;
  static constexpr int kVRow = D + 16;
  static constexpr int kWaveStage = kBlock * (kKRow + kVRow);  // elements per wave
  // LDS pipeline (DMA true): NSD slots per wave, each one block's K
  // then V, 16 unpadded rows of D 16-bit elements with their 16-byte chunks
  // XOR-swizzled by row (the loads place a lane's 16 bytes at a fixed
  // address, so padding is not available).
  static constexpr int kDmaSlotBytes = 2 * kBlock * D * 2;
  // ... followed by a block-table window: two halves of 64 entries.
  static constexpr int kDmaWaveBytes = NSD * kDmaSlotBytes + 2 * 64 * 4;
  static constexpr int kStageBytes = DMA ? W * kDmaWaveBytes : W * kWaveStage * 2;
  static constexpr int kAccBytes = W * NT * (D / 16) * 64 * 16;
  static constexpr int kMlBytes = W * NT * 16 * 2 * 4;
  static constexpr int kBytes =
      kStageBytes > kAccBytes + kMlBytes ? kStageBytes : kAccBytes + kMlBytes;
};

// Whether a segment stages K and V through LDS by direct-to-LDS loads (the
// LDS pipeline) rather than through registers: 16-bit caches at head_dim 128
// with one head tile. FP8 codes must be decoded on the way into LDS, so they
// take registers. Measured on MI355X against the register pipeline (events,
// same tensors, 3 rounds, 32/8/128 fp16 unless noted): B=32 ctx 512 17.96 ->
// 17.34 us, B=64 ctx 512 28.12 -> 27.52, B=64 ctx 4096 164.5 -> 163.2, B=1
// ctx 4096 16.66 -> 16.54, 64/8/128 bf16 B=8 ctx 32768 166.8 -> 165.7, B=8
// ctx 4096 31.56 -> 31.68; two head tiles (ragged MQA) 44.15 -> 45.91, so
// those keep registers.
template <typename KVF, int D, int NT>
constexpr bool dma_staged() {
  return !std::is_same_v<KVF, Fp8E4M3> && D == 128 && NT == 1;
}

// Register pipeline depth: blocks whose K and V are held in VGPRs at once
// (one being processed, the rest in flight); 8 KiB per block at D = 128 with
// a 16-bit cache, 4 KiB with FP8. Measured on MI355X at D = 128: 2 stages
// beat 3..6 for both cache formats (FP8 B=64 ctx 4096: 103 us at 2 stages,
// 107-110 us at 3-6). At D = 64 two head tiles take 4 stages: with 6 the
// balanced kernel needs more than its 256 registers and spills.
template <int D, int NT>
constexpr int mfma_stages() {
  return D <= 64 ? (NT == 2 ? 4 : 6) : 2;
}

// Occupancy floor (waves per SIMD) handed to the register allocator. With two
// head tiles (GQA groups of 17-32) the default allocation lands just above
// the two-wave budget; asking for two keeps the accumulators in VGPRs, no
// spills. Single-tile kernels run best at the allocator's own choice.
template <int D, int NT>
constexpr int mfma_waves_per_eu() {
  return NT == 2 ? 2 : 1;
}

// Row of q (and of the output) that local head hl of unit u reads.
__device__ __forceinline__ int64_t q_row(const DecodeArgs& a, const Unit& u, int hl) {
  return static_cast<int64_t>(u.b + hl / a.q_fold) * a.q_heads + u.kvh * a.q_fold + hl % a.q_fold;
}

// Where a segment's result goes: the normalised output (dtype) when the
// segment covers its whole unit, else an fp32 partial and its log2-sum-exp.
// Local head h (0 .. heads_per_wg-1) of the partial lives at o + h*o_head_stride
// and lse + h*lse_head_stride.
struct Dest {
  bool final;
  float* o;
  float* lse;
  int64_t o_head_stride;
  int lse_head_stride;
};

// Makes the kernel fetch its launch arguments together at entry. The
// compiler loads a kernel argument where it is first needed and waits for each
// such load in turn; the uniform decode kernel's prologue showed three
// dependent argument round trips before its first q load. Naming the fields
// the kernels read as inputs of an empty asm statement has them loaded before
// it, with one wait.
__device__ __forceinline__ void fetch_args(const DecodeArgs& a) {
  asm volatile("" ::"s"(a.q), "s"(a.k), "s"(a.v), "s"(a.out), "s"(a.block_table), "s"(a.seq_lens), "s"(a.o_part),
               "s"(a.lse_part), "s"(a.bt_stride), "s"(a.page_stride), "s"(a.arrivals));
  asm volatile("" ::"s"(a.token_stride), "s"(a.batch), "s"(a.num_q_heads), "s"(a.num_kv_heads), "s"(a.group),
               "s"(a.page_size), "s"(a.bpp_magic), "s"(a.bpp_shift), "s"(a.max_pages), "s"(a.num_splits),
               "s"(a.pages_per_split), "s"(a.head_groups), "s"(a.heads_per_wg), "s"(a.grid), "s"(a.even_start),
               "s"(a.seg_charge), "s"(a.scale_log2),
               "s"(a.q_fold), "s"(a.q_heads), "s"(a.force_partial));
}

// Q as the B operand of S = K Q^T for unit (b, kvh, hg): lane holds head
// h0 + 16t + row, dims 32c + 8grp .. +7 of chunk c (a lane whose head is past
// the group reads the group's first head; mfma_segment zeroes it). It depends
// on the unit alone, not on seq_lens, so a kernel can issue these loads before
// it waits for the sequence length. Nothing here uses the loaded values: the
// compiler's wait for them lands where mfma_segment first does, before its
// main loop.
template <int NT, int KC>
struct QFrag {
  u32x4 v[NT][KC];
};

template <typename E, int D, int NT>
__device__ __forceinline__ void load_q(const DecodeArgs& a, const Unit& u, QFrag<NT, D / 32>& qf) {
  using S = typename E::S;
  const int lane = __lane_id();
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int h0 = u.hg * a.heads_per_wg;
  const S* q = static_cast<const S*>(a.q);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int hl = h0 + 16 * t + row;
    const S* qh = q + q_row(a, u, hl < a.group ? hl : 0) * D;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) qf.v[t][c] = *reinterpret_cast<const u32x4*>(qh + 32 * c + 8 * grp);
  }
}

// Block-table window of one wave of the LDS pipeline (see mfma_segment): half
// h holds the entries of the wave's blocks first + W (64 w + lane) for window
// w = h (mod 2), the lane's block clamped to the wave's last block (nblk of
// them). One 4-byte load per lane straight into LDS.
template <int W>
__device__ __forceinline__ void dma_window_load(const DecodeArgs& a, int* win, int b, int first, int nblk, int w) {
  const int j = min(64 * w + __lane_id(), nblk - 1);
  buffer_load4_lds(a.block_table + static_cast<int64_t>(b) * a.bt_stride, a.max_pages * 4, win + (w & 1) * 64,
                   static_cast<uint32_t>(block_page(a, first + W * j)) * 4u);
}

template <int D, int NT, int W, int NSD>
__device__ __forceinline__ int* dma_window(char* lds, int wave) {
  using Lds = MfmaLds<D, NT, W, true, NSD>;
  return reinterpret_cast<int*>(lds + wave * Lds::kDmaWaveBytes + NSD * Lds::kDmaSlotBytes);
}

// Issues, before seq_lens is known, the first two window halves of this
// wave's part of a segment of sequence b that starts at page page_begin, as
// if the sequence reached page page_cap. mfma_segment with win_ready skips
// its own first window loads: the entries it reads (the sequence's blocks)
// are the same, and entries past its last block are never read. A caller
// that returns without running the segment must wait for these loads first.
template <typename KVF, int D, int NT, int W = kWaves, int NSD = kDmaStages>
__device__ __forceinline__ void prefetch_window(const DecodeArgs& a, char* lds, int b, int page_begin, int page_cap,
                                                int wave) {
  if constexpr (dma_staged<KVF, D, NT>()) {
    const int bpp = a.page_size / kBlock;
    const int first = page_begin * bpp + wave;
    const int blk_cap = page_cap * bpp;
    const int ncap = first < blk_cap ? (blk_cap - first + W - 1) / W : 0;
    int* win = dma_window<D, NT, W, NSD>(lds, wave);
    if (ncap > 0) dma_window_load<W>(a, win, b, first, ncap, 0);
    if (ncap > 64) dma_window_load<W>(a, win, b, first, ncap, 1);
  }
}

// One unit segment on the MFMA path: pages [u.page_begin, u.page_end) of
// KV head u.kvh, head group u.hg of sequence u.b, by all waves of the
// workgroup. Contains two workgroup barriers, reached by every wave; on
// return every wave may still be writing its share of the result, so a caller
// that runs another segment must pass a barrier before touching `lds` again.
//
// KVF is the cache's element format: E itself, or Fp8E4M3, whose codes are
// decoded exactly to E while they are staged into LDS; from there on both
// formats share every instruction. An FP8 cache's per-head scales are folded
// into the score scale (K) and the epilogue (V): q.(s_k k) = s_k (q.k) and
// sum p (s_v v) = s_v sum p v.
//
// qpre: the unit's Q fragments, already loaded by the caller (load_q), or
// null. win_ready: the caller has issued this wave's first block-table window
// loads for this segment (prefetch_window); LDS pipeline only.
template <typename E, typename KVF, int D, int NT, int W = kWaves, int NSD = kDmaStages>
__device__ __forceinline__ void mfma_segment(const DecodeArgs& a, char* lds, const Unit& u, const Dest& dst,
                                             const int wave, const QFrag<NT, D / 32>* qpre = nullptr,
                                             const bool win_ready = false) {
  using S = typename E::S;
  using KS = typename KVF::S;          // cache storage type
  using M = Mfma<E>;
  constexpr bool KV8 = std::is_same_v<KVF, Fp8E4M3>;
  constexpr int KB = KVF::kBytes;      // cache bytes per element
  constexpr int KC = D / 32;           // QK k-chunks
  constexpr int DT = D / 16;           // PV output tiles along head_dim
  constexpr int EPL = 16 / KB;         // cache elements per 16-byte lane load
  constexpr int LPT = D / EPL;         // lanes per token row in a load
  constexpr int TPL = 64 / LPT;        // tokens per load instruction
  constexpr int NL = kBlock / TPL;     // 16-byte loads per lane per block, each of K and V
  static_assert(TPL <= kBlock && kBlock % TPL == 0, "a load must stay inside its 16-token block");
  constexpr bool kDma = dma_staged<KVF, D, NT>();
  using Lds = MfmaLds<D, NT, W, kDma, NSD>;
  constexpr int KROW = Lds::kKRow;
  constexpr int VROW = Lds::kVRow;
  constexpr int NS = mfma_stages<D, NT>();

  const int lane = __lane_id();
  const int row = lane & 15;  // MFMA row / column index of this lane
  const int grp = lane >> 4;  // MFMA k-group of this lane
  const int h0 = u.hg * a.heads_per_wg;

  // Q as the B operand of S = K Q^T (load_q); heads past the group are zero.
  u32x4 qf[NT][KC];
  {
    QFrag<NT, KC> raw;
    if (qpre != nullptr) {
      raw = *qpre;
    } else {
      load_q<E, D, NT>(a, u, raw);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool valid = h0 + 16 * t + row < a.group;
#pragma unroll
      for (int c = 0; c < KC; ++c) qf[t][c] = valid ? raw.v[t][c] : u32x4{0, 0, 0, 0};
    }
  }

  float m[NT], l[NT];
  f32x4 acc[NT][DT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    m[t] = -INFINITY;
    l[t] = 0.0f;
#pragma unroll
    for (int d = 0; d < DT; ++d) acc[t][d] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const KS* kc = static_cast<const KS*>(a.k);
  const KS* vc = static_cast<const KS*>(a.v);
  // Score scale (log2 domain) and output scale of this KV head.
  float qk_scale = a.scale_log2;
  float out_scale = 1.0f;
  if constexpr (KV8) {
    qk_scale *= as_constant(a.k_scale)[u.kvh];
    out_scale = as_constant(a.v_scale)[u.kvh];
  }
  const const_i32_ptr bt = as_constant(a.block_table + static_cast<int64_t>(u.b) * a.bt_stride);
  const int bpp = a.page_size / kBlock;  // blocks per page
  const int blk_begin = u.page_begin * bpp;
  const int blk_end = min(u.page_end * bpp, (u.seq_len + kBlock - 1) / kBlock);
  // This wave's blocks: blk_begin + wave + W * i, i < nblk.
  const int first = blk_begin + wave;
  const int nblk = first < blk_end ? (blk_end - first + W - 1) / W : 0;

  // Per-lane byte offsets inside a block (token row x head dims), for buffer
  // loads off a per-block wave-uniform base. Load c covers tokens
  // c*TPL .. c*TPL + TPL-1; lane l reads 16 bytes (EPL elements) of token
  // c*TPL + l/LPT, head dims v_dim .. v_dim + EPL - 1.
  uint32_t kv_off[NL];
  const int v_tok = lane / LPT;
  const int v_dim = EPL * (lane % LPT);
#pragma unroll
  for (int c = 0; c < NL; ++c) {
    kv_off[c] = static_cast<uint32_t>(((c * TPL + v_tok) * a.token_stride + v_dim) * KB);
  }
  // K and V are both loaded row-coalesced (each 16-lane row reads 256
  // contiguous bytes: a token's head dims), which the memory system streams
  // markedly faster than the MFMA operand layout, and are re-laid out through
  // this wave's LDS tiles: K rows are read back as the A operand (lane = token,
  // 8 dims), V through the transposing read.
  S* kstage = reinterpret_cast<S*>(lds) + wave * Lds::kWaveStage;
  S* stage = kstage + kBlock * KROW;
  const S* k_src = kstage + row * KROW + 8 * grp;
  // Source of this lane's 8-byte chunk in the transposing V^T read: token
  // 4grp + row/4, dims 4(row % 4) .. +3 of each 16-wide tile.
  const S* tr_src = stage + (4 * grp + (row >> 2)) * VROW + 4 * (row & 3);

  // LDS pipeline addressing (kDma). A staged block is 16 rows of D elements
  // whose 16-byte chunks are permuted within each row: token t's chunk c sits
  // in slot c ^ t for K and c ^ 2(t % 8) for V, so that the rows one read
  // phase touches fall on distinct banks (K: 16 rows x 16 bytes; V's
  // transposing read: 4 rows x 4 pieces of 8 bytes). Load c puts lane l's
  // 16 bytes at byte c * 1024 + 16 l, i.e. token 4c + l/16, slot l % 16: the
  // lane reads the chunk that belongs there, and every 16-lane row still
  // reads one whole 256-byte token row from memory. Readers XOR a per-lane
  // base with the chunk's index: the permutation and the index occupy
  // disjoint address bits.
  uint32_t k_off[NL], v_off[NL];
  int k_rd = 0, v_rd = 0;  // element offsets in a slot's K and V rows
  if constexpr (kDma) {
    static_assert(D == 128 && NL == 4 && TPL == 4, "the LDS pipeline is laid out for head_dim 128");
#pragma unroll
    for (int c = 0; c < NL; ++c) {
      const int tok = 4 * c + (lane >> 4);
      const int slot = lane & 15;
      k_off[c] = static_cast<uint32_t>((tok * a.token_stride + (slot ^ tok) * 8) * 2);
      v_off[c] = static_cast<uint32_t>((tok * a.token_stride + (slot ^ (2 * (tok & 7))) * 8) * 2);
    }
    // K as the A operand, chunk c: token `row`, dims 32c + 8grp .. +7.
    k_rd = row * D + ((grp ^ (row & 3)) << 3) + ((row >> 2) << 5);
    // V^T: token 4grp + row/4, dims 16dt + 4(row % 4) .. +3.
    const int tok = 4 * grp + (row >> 2);
    v_rd = tok * D + (((row & 3) >> 1) << 3) + 4 * (row & 1) + ((tok & 7) << 4);
  }

  // Element offset of this wave's i-th block in page `page` (wave-uniform,
  // scalar math).
  auto page_base = [&](int i, int page) -> int64_t {
    const int blk = first + W * i;
    const int pidx = block_page(a, blk);
    return static_cast<int64_t>(page) * a.page_stride +
           static_cast<int64_t>((blk - pidx * bpp) * kBlock) * a.token_stride + static_cast<int64_t>(u.kvh) * D;
  };
  auto block_base = [&](int i) -> int64_t { return page_base(i, bt[block_page(a, first + W * i)]); };
  // The block-table entry of block i by a vector load (every lane reads the
  // same entry). Inside the main loop the entries come this way, not through
  // scalar loads: the LDS reads' waits count scalar loads too (one counter),
  // so a scalar load there made every block wait for the table.
  const auto btr = make_rsrc(a.block_table + static_cast<int64_t>(u.b) * a.bt_stride);
  auto page_load = [&](int i) -> float {
    return buffer_load_f32(btr, static_cast<uint32_t>(block_page(a, first + W * i)) * 4u);
  };

  // A padding slot of the last round (live false) loads through resources of
  // no records: the hardware answers with zeros and touches no memory, so no
  // load is still travelling when the waves meet at the merge's barrier
  // (which waits for every outstanding load).
  auto load_block = [&](int64_t base, u32x4 (&kf)[NL], u32x4 (&vf)[NL], bool live) {
    const int records = live ? 0x7fffffff : 0;
    const auto kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<KS*>(kc + base), static_cast<short>(0), records,
                                                      kBufferDword3);
    const auto vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<KS*>(vc + base), static_cast<short>(0), records,
                                                      kBufferDword3);
#pragma unroll
    for (int c = 0; c < NL; ++c) kf[c] = buffer_load16<kKvPolicy>(kr, kv_off[c]);
#pragma unroll
    for (int c = 0; c < NL; ++c) vf[c] = buffer_load16<kKvPolicy>(vr, kv_off[c]);
  };
  // One 16-byte load's elements into a staging row as E: a plain store for a
  // 16-bit cache, decoded to two 16-byte chunks for FP8.
  auto stage16 = [&](S* dst, u32x4 v) {
    if constexpr (KV8) {
      u32x4 lo, hi;
      fp8x16_to<E>(v, lo, hi);
      *reinterpret_cast<u32x4*>(dst) = lo;
      *reinterpret_cast<u32x4*>(dst + 8) = hi;
    } else {
      *reinterpret_cast<u32x4*>(dst) = v;
    }
  };

  // Scores, online softmax and P V of block i, from its K operand (the A
  // operand of S = K Q^T: lane holds token `row`, dims 32c + 8grp .. +7),
  // a stage_v(nvalid) step run before the V tiles are read, and v_tile(dt),
  // which reads V^T tile dt (lane holds V[token 4grp + j][dim 16dt + row]).
  auto compute_block = [&](int i, const u32x4 (&ka)[KC], auto&& stage_v, auto&& v_tile) {
    // Valid tokens in the block: >= 16 means all; <= 0 only for the padding
    // slots of the last pipeline round (i >= nblk).
    const int nvalid = i < nblk ? u.seq_len - (first + W * i) * kBlock : 0;

    // Scores: lane holds S[token 4grp + i][head row] for tile t.
    u32x2 pf[NT], pl[NT];
    float alpha[NT];
    bool grew = false;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < KC; ++c) s = M::mma(ka[c], qf[t][c], s);
      float sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = s[j] * qk_scale;
      // Only a sequence's last block (and a padding slot) has tokens to mask;
      // nvalid is wave-uniform, so full blocks skip the selects.
      if (nvalid < kBlock) {
#pragma unroll
        for (int j = 0; j < 4; ++j) sc[j] = (4 * grp + j < nvalid) ? sc[j] : -INFINITY;
      }
      float mx = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
      mx = max_xor32(max_xor16(mx));
      // The reference max m moves only when a score passes it by more than
      // kRescaleSlack (log2 units), so the weights p = 2^(s - m) stay below
      // 2^kRescaleSlack and the outputs are rescaled in few blocks rather
      // than in most. Any m gives the same softmax: the outputs, the
      // normaliser and the log-sum-exp all refer to it. A real block's token
      // 0 is valid, so mx is finite; the first block always moves m off
      // -inf; a padding slot has mx = -inf and leaves m as it is.
      const float m_new = mx > m[t] + kRescaleSlack ? mx : m[t];
      grew |= m_new > m[t];
      alpha[t] = __builtin_amdgcn_exp2f(m[t] - m_new);
      float p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) p[j] = __builtin_amdgcn_exp2f(sc[j] - m_new);
      l[t] = l[t] * alpha[t] + ((p[0] + p[1]) + (p[2] + p[3]));
      m[t] = m_new;
      pf[t] = u32x2{pack2<E>(p[0], p[1]), pack2<E>(p[2], p[3])};
      pl[t] = u32x2{pack2_residual<E>(p[0], p[1], pf[t][0]), pack2_residual<E>(p[2], p[3], pf[t][1])};
    }
    // Rescale the outputs only when some head's running max moved (alpha < 1).
    if (__any(grew)) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[t][dt] *= alpha[t];
      }
    }

    stage_v(nvalid);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const u32x2 va = v_tile(dt);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t][dt] = pv_split<E>(va, pf[t], pl[t], acc[t][dt]);
    }
  };

  // Register pipeline: block i's K and V arrive in registers (kf, vf) and are
  // re-laid out through this wave's LDS tile.
  auto process_block = [&](int i, const u32x4 (&kf)[NL], const u32x4 (&vf)[NL]) {
    // Stage K (its rows past seq_len only feed scores replaced by -inf).
#pragma unroll
    for (int c = 0; c < NL; ++c) stage16(kstage + (c * TPL + v_tok) * KROW + v_dim, kf[c]);
    u32x4 ka[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) ka[c] = *reinterpret_cast<const u32x4*>(k_src + 32 * c);
    compute_block(
        i, ka,
        [&](int nvalid) {
          // Stage V, rows past seq_len as zeros, for the transposed reads.
#pragma unroll
          for (int c = 0; c < NL; ++c) {
            const int tok = c * TPL + v_tok;
            stage16(stage + tok * VROW + v_dim, tok < nvalid ? vf[c] : u32x4{0, 0, 0, 0});
          }
        },
        [&](int dt) { return lds_read_tr16(tr_src + 16 * dt); });
  };

  // LDS pipeline: block i's K and V load straight into its LDS slot (rows
  // past seq_len as zeros); K and then V are waited for just before they are
  // read (the loop's issue order makes both waits exact: see there).
  auto process_block_lds = [&](int i, const char* slot, auto&& wait_k, auto&& wait_v) {
    const S* ks = reinterpret_cast<const S*>(slot);
    const S* vs = ks + kBlock * D;
    wait_k();
    u32x4 ka[KC];
#pragma unroll
    for (int c = 0; c < KC; ++c) ka[c] = *reinterpret_cast<const u32x4*>(ks + (k_rd ^ (c << 5)));
    compute_block(i, ka, [&](int) { wait_v(); }, [&](int dt) { return lds_read_tr16(vs + (v_rd ^ (dt << 4))); });
  };

  if constexpr (kDma) {
    if (nblk > 0) {
      // LDS pipeline, NSD deep: while block i is processed from
      // its slot, blocks i+1 .. i+NSD-1 are loading straight into theirs.
      // Each iteration issues 8 of these loads (block i + NSD - 1's 4 for K,
      // then 4 for V; asm statements keep their order), which the compiler
      // does not see, and they complete in order: once at most
      // 8 (NSD - 1) + 4 are in flight, block i's K is in LDS, and its V once
      // at most 8 (NSD - 1) are. (An iteration that also refills the
      // block-table window issues one more load, first, which only makes
      // these waits stricter.)
      //
      // Block-table entries come the same way, into a window in LDS: half h
      // holds the entries of blocks 64w .. 64w + 63 for w = h (mod 2), one per
      // lane of a 4-byte load, and is refilled with w + 2 when the loop
      // enters window w + 1, 64 blocks before it is read. With no vector load
      // the compiler can see inside the loop, it adds no waits there.
      char* slots = lds + wave * Lds::kDmaWaveBytes;
      int* win = dma_window<D, NT, W, NSD>(lds, wave);
      auto window_load = [&](int w) { dma_window_load<W>(a, win, u.b, first, nblk, w); };
      if (!win_ready) {
        window_load(0);
        if (nblk > 64) window_load(1);
      }
      wait_vmcnt<0>();  // the first window is read right away (q's loads land too)
      auto dma_block = [&](int j, int slot, int valid) {
        if (j >= 64 && (j & 63) == 0 && 64 * ((j >> 6) + 1) < nblk) window_load((j >> 6) + 1);
        const int page = __builtin_amdgcn_readfirstlane(win[((j >> 6) & 1) * 64 + (j & 63)]);
        const int64_t off = page_base(j, page);
        const int records = valid > 0 ? min(valid, kBlock) * a.token_stride * 2 : 0;
        char* dst = slots + slot * Lds::kDmaSlotBytes;
#pragma unroll
        for (int c = 0; c < NL; ++c) buffer_load16_lds_nt(kc + off, records, dst + c * 1024, k_off[c]);
#pragma unroll
        for (int c = 0; c < NL; ++c) buffer_load16_lds_nt(vc + off, records, dst + kBlock * D * 2 + c * 1024, v_off[c]);
      };
      auto valid_of = [&](int i) { return i < nblk ? u.seq_len - (first + W * i) * kBlock : 0; };
#pragma unroll
      for (int k = 0; k < NSD - 1; ++k) dma_block(min(k, nblk - 1), k, valid_of(k));
      for (int base = 0; base < nblk; base += NSD) {
#pragma unroll
        for (int s = 0; s < NSD; ++s) {
          const int i = base + s;
          dma_block(min(i + NSD - 1, nblk - 1), (s + NSD - 1) % NSD, valid_of(i + NSD - 1));
          process_block_lds(i, slots + s * Lds::kDmaSlotBytes, [] { wait_vmcnt<8 * (NSD - 1) + 4>(); },
                            [] { wait_vmcnt<8 * (NSD - 1)>(); });
        }
      }
      // The last round's loads past the end write zeros into slots that the
      // cross-wave merge below reuses: let them land first.
      wait_vmcnt<0>();
    } else if (win_ready) {
      // A wave with no block of this segment still has the caller's window
      // loads in flight into LDS that the cross-wave merge reuses.
      wait_vmcnt<0>();
    }
  } else if (nblk > 0) {
    // NS-stage pipeline: while block i is processed, blocks i+1 .. i+NS-1 are
    // in flight. The loop runs a whole number of NS-block rounds with no
    // branch inside, so the compiler's load-wait counts stay exact; slots past
    // the last block re-read the last block (cache-resident) and process it
    // with no valid token, which leaves the running state unchanged.
    //
    // Block-table entries run NS blocks ahead of the K/V loads, in a ring of
    // NS: iteration i turns the entry of block i + NS - 1 (loaded at
    // iteration i - NS) into the address of that block's K/V loads, then
    // loads the entry of block i + 2NS - 1 into the freed slot ahead of those
    // K/V loads. Vector loads complete in order, so the wait for block
    // i + NS - 1's K/V (in iteration i + NS - 1) also covers that entry before
    // iteration i + NS uses it: the table costs the loop no wait of its own.
    // The ring's first entries are loaded before the first blocks' K/V, as
    // in the loop: the compiler sizes its waits for the worst path into the
    // loop, and entries loaded after those K/V would make it wait for them on
    // every iteration.
    u32x4 kb[NS][NL], vb[NS][NL];
    float pg[NS];  // entry bits of blocks i + NS - 1 .. i + 2NS - 2, slot = block % NS
#pragma unroll
    for (int k = NS - 1; k < 2 * NS - 1; ++k) pg[k % NS] = page_load(min(k, nblk - 1));
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) load_block(block_base(min(s, nblk - 1)), kb[s], vb[s], s < nblk);
    for (int base = 0; base < nblk; base += NS) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const int i = base + s;
        const int slot = (s + NS - 1) % NS;  // block i + NS - 1 (base is a multiple of NS)
        const int j = min(i + NS - 1, nblk - 1);
        const int64_t nb = page_base(j, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, pg[slot])));
        pg[slot] = page_load(min(i + 2 * NS - 1, nblk - 1));
        load_block(nb, kb[slot], vb[slot], i + NS - 1 < nblk);
        process_block(i, kb[s], vb[s]);
      }
    }
  }

  // Per-wave normaliser: the four lane groups hold disjoint tokens of a head.
#pragma unroll
  for (int t = 0; t < NT; ++t) l[t] = sum_xor32(sum_xor16(l[t]));

  // Cross-wave merge, shared by the waves. Every wave publishes its running
  // max and normaliser and all of its output tiles in LDS; then wave w
  // combines the output chunks (t, dt) with t * DT + dt = w (mod W) from all
  // W waves by the log-sum-exp rule and writes them. Measured on MI355X, the
  // one-wave form of this merge (wave 0 reading everyone's tiles, the others
  // idle) took 2.2 us per segment at one head tile and 3.8 us at two.
  // Contributions are added in wave order 0 .. W-1 whichever wave combines
  // them. The staging tiles are reused, so every wave must have left the main
  // loop first.
  __syncthreads();
  f32x4* lds_acc = reinterpret_cast<f32x4*>(lds);  // [W][NT * DT][64 lanes]
  float* lds_ml = reinterpret_cast<float*>(lds_acc + W * NT * DT * 64);
  if (lane < 16) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      lds_ml[((wave * NT + t) * 16 + lane) * 2 + 0] = m[t];
      lds_ml[((wave * NT + t) * 16 + lane) * 2 + 1] = l[t];
    }
  }
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) lds_acc[(wave * NT * DT + t * DT + dt) * 64 + lane] = acc[t][dt];
  }
  __syncthreads();

#pragma unroll
  for (int t = 0; t < NT; ++t) {
    float mw[W], lw[W];
    float mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = lds_ml[((w * NT + t) * 16 + row) * 2 + 0];
      lw[w] = lds_ml[((w * NT + t) * 16 + row) * 2 + 1];
      mmax = fmaxf(mmax, mw[w]);
    }
    // Weights 2^(m_w - max) lie in [0, 1]: the hardware exponential suffices
    // (one whose result is denormal contributes nothing visible).
    float cw[W];
    float denom = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      cw[w] = mw[w] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw[w] - mmax);
      denom += lw[w] * cw[w];
    }
    const float inv = out_scale / denom;
    const int hl = h0 + 16 * t + row;
    const bool valid = hl < a.group;
    const int64_t head = q_row(a, u, valid ? hl : 0);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      if ((t * DT + dt) % W != wave) continue;  // another wave's chunk
      f32x4 num = lds_acc[(t * DT + dt) * 64 + lane] * cw[0];
#pragma unroll
      for (int w = 1; w < W; ++w) num += lds_acc[(w * NT * DT + t * DT + dt) * 64 + lane] * cw[w];
      float o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = num[i] * inv;
      if (!valid) continue;
      const int d = 16 * dt + 4 * grp;
      if (dst.final) {
        S* out = static_cast<S*>(a.out) + head * D + d;
        *reinterpret_cast<u32x2*>(out) = u32x2{pack2<E>(o[0], o[1]), pack2<E>(o[2], o[3])};
      } else {
        // Partials are stored device-coherent: with the fused merge, a
        // workgroup on another XCD reads them within this launch.
        const uint32_t off = static_cast<uint32_t>((static_cast<int64_t>(16 * t + row) * dst.o_head_stride + d) * 4);
        buffer_store16<kCachePolicyDevice>(make_rsrc(uniform_ptr(dst.o)), off,
                                           __builtin_bit_cast(u32x4, f32x4{o[0], o[1], o[2], o[3]}));
      }
    }
    // The log2-sum-exp of tile t comes from the wave that combines its chunk 0.
    if (valid && !dst.final && grp == 0 && (t * DT) % W == wave) {
      buffer_store_f32<kCachePolicyDevice>(make_rsrc(uniform_ptr(dst.lse)),
                                           static_cast<uint32_t>((16 * t + row) * dst.lse_head_stride * 4),
                                           mmax + __builtin_amdgcn_logf(denom));
    }
  }
}

// ------------------------------------------------------- fused split merge
//
// A unit split across several segments (uniform splits, or a balanced
// workgroup range) is merged by whichever of its segments finishes last, in
// the decode kernel itself, instead of by a separate merge launch (measured
// at 4.0-5.5 us per call on MI355X). Each segment that wrote a partial
// publishes it (release fence) and adds one to its unit's arrival counter;
// the one that brings the counter to the unit's segment count resets it to
// zero, acquires the others' partials and merges them with merge_partials,
// so the result is bit-identical to the merge kernels'. Nobody waits, so a
// missing arrival cannot hang a workgroup.
//
// The counters live in device memory owned by the library, zero when the
// code object is loaded and zero again after every completed call (the last
// arriver of each unit resets its counter). Calls whose kernels may overlap
// must not share counters, so a call takes a region that only calls ordered
// with it use (arrival_region): an eager call the region of its stream
// (kernels on one stream never overlap), a call recorded into a graph a
// region of its own capture sequence and capture stream, never shared with
// eager streams or other captures. With the regions of a kind used up, or on
// a per-thread default stream (one handle, many streams), the call takes the
// merge kernel; results are bit-identical either way.
constexpr int kStreamRegions = 64;       // eager streams served per device
constexpr int kCaptureRegions = 192;     // captured (capture sequence, stream) pairs per device
constexpr int kArrivalRegions = kStreamRegions + kCaptureRegions;
constexpr int kArrivalCounters = 8192;   // units per region (8 MiB per device in all)
// Query heads of a fused unit (one head tile, at most two heads per wave).
// Measured on MI355X for MQA units (32 heads, two head tiles): the last
// arriver's 8-heads-per-wave merge made the ragged 64-sequence batch slower
// than the merge kernel (52.4 vs 49.8 us), and the merge code alone slowed
// the two-tile kernel's main loop (46 -> 50 us), so those keep the merge kernel.
constexpr int kFusedMergeMaxHeads = 8;
// The last arriver's four waves merge the unit serially: each takes
// cdiv(heads, 4) heads of `segments` partials, where the merge kernel gives
// every (sequence, head) its own wave. Measured on MI355X (events, us, same
// uniform splits, fused vs merge kernel), by heads per wave x segments: 8-16
// mostly faster (64/8/128 B=1 ctx 4096 S=8 15.1 vs 15.8, 8/1/128 B=8 ctx
// 4096 S=8 14.3 vs 15.0, 32/8/128 B=1 ctx 8192 S=16 16.2 vs 16.7; with 16
// short segments slower: 32/8/128 B=2 ctx 2048 S=16 14.1 vs 12.8), 32
// slower (32/8/128 B=1 ctx 4096 S=32 15.2 vs 13.2, B=2 S=32 20.9 vs 15.8,
// 64/8/128 B=1 S=16 14.8 vs 13.6), 64-512 slower still (8/1/128 B=1 ctx
// 8192 22.6 vs 18.1, 32/4/128 B=1 ctx 32768 31.9 vs 28.0): few units split
// over the whole device keep the merge kernel.
constexpr int kFusedMergeMaxWork = 16;

__device__ uint32_t g_decode_arrivals[kArrivalRegions * kArrivalCounters];

template <typename E, int kG = 16, int POL = 0>
__device__ __forceinline__ void merge_partials(const float* lse, int64_t l_stride, const float* op,
                                               int64_t o_stride, int n, int head_dim, typename E::S* out);

// One head's merge inputs, loaded ahead of its reduction (head_merge_load).
template <int kG>
struct HeadMerge {
  f32x4 v[kG];
  float lw[kG];
  float ll;  // lse of row `lane`, -inf past n
};
template <int kG, int POL>
__device__ __forceinline__ void head_merge_load(HeadMerge<kG>& m, const float* lse, int64_t l_stride, const float* op,
                                                int64_t o_stride, int n, int head_dim);
template <typename E, int kG>
__device__ __forceinline__ void head_merge_finish(const HeadMerge<kG>& m, int n, int head_dim, typename E::S* out);

// The partials of one unit: head hl's n partials (lse at lse + hl *
// lse_head_stride + w * l_stride, rows at o + hl * o_head_stride + w *
// o_stride) merge into out + hl * head_dim.
struct MergeJob {
  const float* lse;
  int64_t lse_head_stride, l_stride;
  const float* o;
  int64_t o_head_stride, o_stride;
  int n;      // partials per head (the unit's segments)
  int heads;  // query heads of the unit
  void* out;
};

// Called by every wave of the segment's waves after a segment that wrote a
// partial (each wave wrote its share of it). Two workgroup barriers, reached
// by every wave of the workgroup: paired halves call it together.
//
// Release: the waves stored the partial device-coherent (sc1); each waits for
// its own stores to complete, the barrier orders all of them before wave 0's
// device-scope add, so they are visible to whoever sees the add. Acquire: the
// last arriver reads the partials with device-coherent loads, issued only
// after the add returned.
template <typename E, int W = kWaves>
__device__ void arrive_and_merge(uint32_t* counter, const MergeJob& job, int head_dim, int wave, int* s_last) {
  wait_vector_memory();
  __syncthreads();
  if (wave == 0 && __lane_id() == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old + 1 == static_cast<uint32_t>(job.n);
    // Every arrival has happened: leave the counter zero for the next call.
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_last = last;
  }
  __syncthreads();
  const int last = __builtin_amdgcn_readfirstlane(*s_last);
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");  // no load moves above the arrival
  using S = typename E::S;
  S* out = static_cast<S*>(job.out);
  constexpr int kG = 4;  // rows per lane: one round holds kG * 256 / head_dim partials
  if (job.n <= 64 && job.n <= kG * (256 / head_dim)) {
    // Heads wave, wave + W, ...: the next head's loads are in flight while
    // this one is reduced, so a wave with several heads (a 32-head MQA unit)
    // waits for memory about once.
    HeadMerge<kG> cur, nxt;
    int h = wave;
    if (h < job.heads) {
      head_merge_load<kG, kCachePolicyDevice>(cur, job.lse + h * job.lse_head_stride, job.l_stride,
                                              job.o + h * job.o_head_stride, job.o_stride, job.n, head_dim);
    }
    for (; h < job.heads; h += W) {
      const int hn = h + W;
      if (hn < job.heads) {
        head_merge_load<kG, kCachePolicyDevice>(nxt, job.lse + hn * job.lse_head_stride, job.l_stride,
                                                job.o + hn * job.o_head_stride, job.o_stride, job.n, head_dim);
      }
      head_merge_finish<E, kG>(cur, job.n, head_dim, out + static_cast<int64_t>(h) * head_dim);
      cur = nxt;
    }
  } else {
    for (int h = wave; h < job.heads; h += W) {
      merge_partials<E, 4, kCachePolicyDevice>(job.lse + h * job.lse_head_stride, job.l_stride,
                                               job.o + h * job.o_head_stride, job.o_stride, job.n, head_dim,
                                               out + static_cast<int64_t>(h) * head_dim);
    }
  }
}

// Segments (splits with pages) of a uniform-split unit.
__device__ __forceinline__ int active_splits(const DecodeArgs& a, const Unit& u) {
  const int num_pages = u.seq_len > 0 ? (u.seq_len + a.page_size - 1) / a.page_size : 0;
  return min(a.num_splits, (num_pages + a.pages_per_split - 1) / a.pages_per_split);
}

// The merge of a uniform-split unit: partial w is split w of the unit's heads
// in o_part [batch, num_q_heads, num_splits, head_dim].
template <typename E>
__device__ __forceinline__ MergeJob uniform_job(const DecodeArgs& a, const Unit& u, int head_dim, int n) {
  const int h0 = u.hg * a.heads_per_wg;
  const int64_t head0 = static_cast<int64_t>(u.b) * a.num_q_heads + u.kvh * a.group + h0;
  MergeJob j;
  j.lse = a.lse_part + head0 * a.num_splits;
  j.lse_head_stride = a.num_splits;
  j.l_stride = 1;
  j.o = a.o_part + head0 * a.num_splits * head_dim;
  j.o_head_stride = static_cast<int64_t>(a.num_splits) * head_dim;
  j.o_stride = head_dim;
  j.n = n;
  j.heads = min(a.heads_per_wg, a.group - h0);
  j.out = static_cast<typename E::S*>(a.out) + head0 * head_dim;
  return j;
}

__device__ __forceinline__ uint32_t* unit_counter(const DecodeArgs& a, const Unit& u) {
  return a.arrivals + (static_cast<int64_t>(u.b) * a.num_kv_heads + u.kvh) * a.head_groups + u.hg;
}

// Output of a uniform-split unit: the final output with one split, else its
// split's slot of o_part [batch, num_q_heads, num_splits, head_dim] and
// lse_part [batch, num_q_heads, num_splits].
// With the fused merge, a unit whose sequence reaches only one split writes
// its output directly (bit-identical: a single partial merges to itself).
__device__ __forceinline__ Dest uniform_dest(const DecodeArgs& a, const Unit& u, int head_dim) {
  Dest dst;
  dst.final = !a.force_partial && (a.num_splits == 1 || (a.arrivals != nullptr && active_splits(a, u) == 1));
  const int64_t head0 = static_cast<int64_t>(u.b) * a.num_q_heads + u.kvh * a.group + u.hg * a.heads_per_wg;
  dst.o = dst.final ? nullptr : a.o_part + (head0 * a.num_splits + u.split) * head_dim;
  dst.lse = dst.final ? nullptr : a.lse_part + head0 * a.num_splits + u.split;
  dst.o_head_stride = static_cast<int64_t>(a.num_splits) * head_dim;
  dst.lse_head_stride = a.num_splits;
  return dst;
}

// Uniform splits: workgroup = (sequence, KV head, head group, split), the
// split owning pages_per_split pages (the reference's decomposition).
template <typename E, typename KVF, int D, int NT>
__global__ void __launch_bounds__(kThreads, (mfma_waves_per_eu<D, NT>())) decode_mfma_kernel(const DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[MfmaLds<D, NT, kWaves, dma_staged<KVF, D, NT>()>::kBytes];
  __shared__ int s_last[1];
  fetch_args(a);
  // q and the first block-table window depend on the unit alone: they are
  // issued before the kernel waits for seq_lens, so the first K/V loads
  // follow one memory round trip after it instead of two.
  Unit u = decode_unit_ids(a);
  const int wave = wave_id();
  QFrag<NT, D / 32> q;
  load_q<E, D, NT>(a, u, q);
  const int pb = u.split * a.pages_per_split;
  prefetch_window<KVF, D, NT>(a, lds, u.b, pb, min(pb + a.pages_per_split, a.max_pages), wave);
  unit_pages(a, u);
  if (u.page_begin >= u.page_end) {
    wait_vmcnt<0>();  // the window loads write this workgroup's LDS
    if (u.split == 0 && u.seq_len <= 0 && (a.num_splits == 1 || a.arrivals != nullptr) && !a.force_partial) {
      write_zero_heads<typename E::S, E>(a, u, D, threadIdx.x, blockDim.x);
    }
    return;  // a split past the end of its sequence has no work
  }
  const Dest dst = uniform_dest(a, u, D);
  mfma_segment<E, KVF, D, NT>(a, lds, u, dst, wave, &q, true);
  if constexpr (NT == 1) {  // see kFusedMergeMaxHeads
    if (!dst.final && a.arrivals != nullptr) {
      arrive_and_merge<E>(unit_counter(a, u), uniform_job<E>(a, u, D, active_splits(a, u)), D, wave_id(), s_last);
    }
  }
}

// Uniform splits, two units per 8-wave workgroup: waves 0-3 take KV head 2j
// and waves 4-7 KV head 2j+1 of the same sequence, head group and split
// (decode_unit_paired), each half with its own LDS. The two halves run the
// same segment code as decode_mfma_kernel; together they read 2 adjacent
// head slices (512 contiguous bytes at head_dim 128, 16-bit) of every token
// row at about the same time. Measured on MI355X with the decode's own
// gather as pure loads (B=64, 32/8/128/16 fp16): 6.8 TB/s against 6.5 TB/s
// for one head per 4-wave workgroup; pairing two sequences' units instead
// gains nothing, so the gain is the adjacent-head locality, not the larger
// workgroup.
template <typename E, typename KVF, int D, int NT>
__global__ void __launch_bounds__(2 * kThreads, (mfma_waves_per_eu<D, NT>()))
    decode_mfma_paired_kernel(const DecodeArgs a) {
  using Lds = MfmaLds<D, NT, kWaves, dma_staged<KVF, D, NT>()>;
  __shared__ __attribute__((aligned(16))) char lds[2 * Lds::kBytes];
  __shared__ int s_last[2];
  const int wave = wave_id();
  const int half = wave / kWaves;
  // Both halves hold the same sequence and split, so they agree on whether
  // there is work, whether it is final and how many segments the unit has:
  // they pass the same workgroup barriers.
  fetch_args(a);
  // q and the first block-table window before seq_lens (decode_mfma_kernel).
  Unit u = decode_unit_paired_ids(a, half);
  QFrag<NT, D / 32> q;
  load_q<E, D, NT>(a, u, q);
  const int pb = u.split * a.pages_per_split;
  prefetch_window<KVF, D, NT>(a, lds + half * Lds::kBytes, u.b, pb, min(pb + a.pages_per_split, a.max_pages),
                              wave - half * kWaves);
  unit_pages(a, u);
  if (u.page_begin >= u.page_end) {
    wait_vmcnt<0>();  // the window loads write this workgroup's LDS
    // The other half's segment passes two workgroup barriers: pass them too.
    __syncthreads();
    __syncthreads();
    if (u.split == 0 && u.seq_len <= 0 && (a.num_splits == 1 || a.arrivals != nullptr) && !a.force_partial) {
      write_zero_heads<typename E::S, E>(a, u, D, threadIdx.x - half * kThreads, kThreads);
    }
    return;
  }
  const Dest dst = uniform_dest(a, u, D);
  mfma_segment<E, KVF, D, NT>(a, lds + half * Lds::kBytes, u, dst, wave - half * kWaves, &q, true);
  if constexpr (NT == 1) {  // see kFusedMergeMaxHeads
    if (!dst.final && a.arrivals != nullptr) {
      arrive_and_merge<E>(unit_counter(a, u), uniform_job<E>(a, u, D, active_splits(a, u)), D, wave - half * kWaves,
                          s_last + half);
    }
  }
}

// ------------------------------------------------------- balanced schedule
//
// Work list: every (sequence b, KV head, head group) unit is cdiv(L_b, page
// size) pages long; units are laid end to end, b-major. Workgroup w takes
// positions [w*per, (w+1)*per) of that list, per = max(8, cdiv(total, grid)),
// which may span the tail of one unit and the head of the next, so every
// workgroup streams the same number of pages however uneven the lengths are.
// Totals and prefix sums come from seq_lens on the device (no host sync).
// A unit covered by one workgroup gets its output written directly; a unit
// split across workgroups w0..w1 gets partials in slots w + unit (unique:
// both ranges and units are ordered), merged by decode_merge_balanced_kernel.

__device__ __forceinline__ int seq_pages(const DecodeArgs& a, int b) {
  const int raw = a.seq_lens[b];
  const int64_t cap = static_cast<int64_t>(a.max_pages) * a.page_size;
  const int len = static_cast<int>(raw < cap ? raw : cap);
  return len > 0 ? (len + a.page_size - 1) / a.page_size : 0;
}

// seq_pages for a wave-uniform b: one scalar load.
__device__ __forceinline__ int seq_pages_uniform(const DecodeArgs& a, int b) {
  const int raw = as_constant(a.seq_lens)[b];
  const int64_t cap = static_cast<int64_t>(a.max_pages) * a.page_size;
  const int len = static_cast<int>(raw < cap ? raw : cap);
  return len > 0 ? (len + a.page_size - 1) / a.page_size : 0;
}

__device__ __forceinline__ int wave_incl_scan(int v) { return wave_prefix_sum(v); }

__device__ __forceinline__ int64_t balanced_per(const DecodeArgs& a, int64_t total) {
  return max(static_cast<int64_t>(kMinPagesPerBalancedWg), (total + a.grid - 1) / a.grid);
}

// Pages in the whole work list. Wave-uniform; every wave computes it.
__device__ __forceinline__ int64_t list_total(const DecodeArgs& a, int units_per_seq) {
  const int lane = __lane_id();
  int64_t total = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int b = b0 + lane;
    const int pl = b < a.batch ? seq_pages(a, b) * units_per_seq : 0;
    total += __builtin_amdgcn_readlane(wave_incl_scan(pl), 63);
  }
  return total;
}

// Batches of up to 64 * kScanChunks sequences are scanned with all their
// seq_lens loads in flight at once: one memory round trip at the start.
constexpr int kScanChunks = 4;

// The balanced work list. Each pages-bearing sequence contributes
// units_per_seq units in order; a unit takes charge + n list positions, the
// charge first (no pages: the cut's cost of starting a segment there) and
// then its n pages. charge is a.seg_charge for a batch of at most 64 *
// kScanChunks sequences whose page counts are not all equal, else 0 (an
// even batch's units are cut at their own boundaries already, and a charge
// would only take pages from the workgroups that start a unit). Workgroup w
// takes list positions [w * per, (w + 1) * per).
//
// Length of the work list, the list position where sequence b's units begin,
// sequence b's page count and the charge (b wave-uniform), as the balanced
// kernel's schedule_start computes them.
__device__ __forceinline__ void list_prefix(const DecodeArgs& a, int units_per_seq, int b, int64_t* total,
                                            int64_t* base, int* pages, int* charge) {
  const int lane = __lane_id();
  int64_t t = 0, pre = 0;
  int own = 0, seqs = 0, seqs_before = 0;
  const int n0 = seq_pages(a, 0);
  bool differ = n0 == 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int bb = b0 + lane;
    const int np = bb < a.batch ? seq_pages(a, bb) : 0;
    differ |= bb < a.batch && np != n0;
    const int pl = np * units_per_seq;
    const int incl = wave_incl_scan(pl);
    const uint64_t bearing = __ballot(np > 0);
    if (b >= b0 && b < b0 + 64) {
      pre = t + __builtin_amdgcn_readlane(incl - pl, b - b0);
      own = __builtin_amdgcn_readlane(np, b - b0);
      seqs_before = seqs + __builtin_popcountll(bearing & ((1ull << (b - b0)) - 1));
    }
    t += __builtin_amdgcn_readlane(incl, 63);
    seqs += __builtin_popcountll(bearing);
  }
  const int c = a.batch <= 64 * kScanChunks && __ballot(differ) != 0 ? a.seg_charge : 0;
  *total = t + static_cast<int64_t>(c) * units_per_seq * seqs;
  *base = pre + static_cast<int64_t>(c) * units_per_seq * seqs_before;
  *pages = own;
  *charge = c;
}

// Where workgroup `wg` starts: its first list position `pos` (wg * per), the
// first pages-bearing sequence whose units hold it (batch when pos is past the
// end) and the list position where that sequence's units begin. One pass over
// seq_lens when the batch fits a wave, two otherwise. All results uniform.
struct Start {
  int64_t total, per, pos, base;
  int b;
  int pages;   // pages of sequence b (when b < batch)
  int len;     // its length, clamped to max_pages * page_size
  int charge;  // list positions ahead of each unit's pages (list_prefix)
  // batch <= 64 * kScanChunks only: bit j of empties[k] marks sequence
  // 64 * k + j as existing, without pages, and zeroed by this workgroup
  // (sequence b belongs to workgroup b % grid: the grid may be smaller than
  // the batch when contexts are short).
  uint64_t empties[kScanChunks];
};

__device__ __forceinline__ int clamped_len(const DecodeArgs& a, int raw) {
  const int64_t cap = static_cast<int64_t>(a.max_pages) * a.page_size;
  return static_cast<int>(raw < cap ? raw : cap);
}

__device__ __forceinline__ int pages_of(const DecodeArgs& a, int len) {
  return len > 0 ? (len + a.page_size - 1) / a.page_size : 0;
}

// seq_lens of a batch of at most 64 * kScanChunks sequences: lane l of chunk
// k holds sequence 64k + l (0 past the batch). All chunks' loads are issued
// before any is used, through a resource that ends with the array, so lanes
// past the batch read 0 with no branch. (A per-lane branch around each load,
// with its clamp inside, made the compiler wait for each load in turn: one
// memory round trip per 64 sequences.) Chunks past the batch are skipped by
// uniform branches.
struct LenChunks {
  int raw[kScanChunks];
};

__device__ __forceinline__ LenChunks load_len_chunks(const DecodeArgs& a) {
  const int lane = __lane_id();
  const auto lens_rsrc = make_rsrc_bytes(uniform_ptr(a.seq_lens), static_cast<uint32_t>(a.batch) * 4u);
  LenChunks c;
#pragma unroll
  for (int k = 0; k < kScanChunks; ++k) {
    c.raw[k] = 0;
    if (64 * k < a.batch) {
      c.raw[k] = __builtin_bit_cast(int, buffer_load_f32(lens_rsrc, static_cast<uint32_t>((64 * k + lane) * 4)));
    }
  }
  return c;
}

// The page count every sequence of the batch has (batch <= 64 *
// kScanChunks), or 0 when two sequences differ or sequence 0 has no page.
// One compare per lane and chunk: a length has n pages exactly when it lies
// in ((n - 1) * page_size, n * page_size].
__device__ __forceinline__ int even_pages(const DecodeArgs& a, const LenChunks& c) {
  const int lane = __lane_id();
  const int n = pages_of(a, clamped_len(a, __builtin_amdgcn_readfirstlane(c.raw[0])));
  const int64_t lo = static_cast<int64_t>(n - 1) * a.page_size;  // exclusive
  const int64_t hi = static_cast<int64_t>(n) * a.page_size;
  bool differ = false;
#pragma unroll
  for (int k = 0; k < kScanChunks; ++k) {
    if (64 * k < a.batch) {
      const int len = clamped_len(a, c.raw[k]);
      differ |= 64 * k + lane < a.batch && (len <= lo || len > hi);
    }
  }
  return n > 0 && __ballot(differ) == 0 ? n : 0;
}

// The clamped length of sequence b (wave-uniform, b < batch <= 64 *
// kScanChunks), read from the lanes that loaded it.
__device__ __forceinline__ int chunk_len(const DecodeArgs& a, const LenChunks& c, int b) {
  int raw = 0;
#pragma unroll
  for (int k = 0; k < kScanChunks; ++k) {
    if ((b >> 6) == k) raw = __builtin_amdgcn_readlane(c.raw[k], b & 63);
  }
  return clamped_len(a, raw);
}

// c: the batch's seq_lens (load_len_chunks) when batch <= 64 * kScanChunks.
__device__ __forceinline__ Start schedule_start(const DecodeArgs& a, int units_per_seq, int wg, const LenChunks& c) {
  const int lane = __lane_id();
  Start s;
#pragma unroll
  for (int k = 0; k < kScanChunks; ++k) s.empties[k] = 0;
  s.pages = 0;
  s.len = 0;
  s.charge = 0;
  if (a.batch <= 64 * kScanChunks) {
    s.charge = even_pages(a, c) > 0 ? 0 : a.seg_charge;
    int len[kScanChunks], pl[kScanChunks], incl[kScanChunks];
    int64_t before[kScanChunks];
#pragma unroll
    for (int k = 0; k < kScanChunks; ++k) len[k] = clamped_len(a, c.raw[k]);
    int64_t total = 0;
#pragma unroll
    for (int k = 0; k < kScanChunks; ++k) {
      pl[k] = 0;
      incl[k] = 0;
      before[k] = total;
      if (64 * k < a.batch) {
        const int np = pages_of(a, len[k]);
        pl[k] = np > 0 ? (np + s.charge) * units_per_seq : 0;
        incl[k] = wave_incl_scan(pl[k]);
        total += __builtin_amdgcn_readlane(incl[k], 63);
        const int b = 64 * k + lane;
        s.empties[k] = __ballot(b < a.batch && pl[k] == 0 && b % a.grid == static_cast<int>(blockIdx.x));
      }
    }
    s.total = total;
    s.per = balanced_per(a, s.total);
    s.pos = static_cast<int64_t>(wg) * s.per;
    s.b = a.batch;
    s.base = s.total;
    bool found = false;
#pragma unroll
    for (int k = 0; k < kScanChunks; ++k) {
      if (!found && 64 * k < a.batch && before[k] + __builtin_amdgcn_readlane(incl[k], 63) > s.pos) {
        const int j = __builtin_ctzll(__ballot(before[k] + incl[k] > s.pos));
        s.b = 64 * k + j;
        s.base = before[k] + __builtin_amdgcn_readlane(incl[k] - pl[k], j);
        s.pages = __builtin_amdgcn_readlane(pl[k], j) / units_per_seq - s.charge;
        s.len = __builtin_amdgcn_readlane(len[k], j);
        found = true;
      }
    }
  } else {
    s.total = list_total(a, units_per_seq);
    s.per = balanced_per(a, s.total);
    s.pos = static_cast<int64_t>(wg) * s.per;
    s.b = a.batch;
    s.base = 0;
    for (int b0 = 0; b0 < a.batch; b0 += 64) {
      const int b = b0 + lane;
      const int len = b < a.batch ? clamped_len(a, a.seq_lens[b]) : 0;
      const int pl = pages_of(a, len) * units_per_seq;
      const int incl = wave_incl_scan(pl);
      const int chunk = __builtin_amdgcn_readlane(incl, 63);
      if (s.base + chunk > s.pos) {
        const int j = __builtin_ctzll(__ballot(s.base + incl > s.pos));
        s.b = b0 + j;
        s.base += __builtin_amdgcn_readlane(incl - pl, j);
        s.pages = __builtin_amdgcn_readlane(pl, j) / units_per_seq;
        s.len = __builtin_amdgcn_readlane(len, j);
        break;
      }
      s.base += chunk;
    }
  }
  s.b = __builtin_amdgcn_readfirstlane(s.b);
  s.pages = __builtin_amdgcn_readfirstlane(s.pages);
  s.len = __builtin_amdgcn_readfirstlane(s.len);
  s.charge = __builtin_amdgcn_readfirstlane(s.charge);
  return s;
}

// A balanced-schedule workgroup (one per CU, or one per CU and KV-head pair)
// has kWaves waves per KV head. Measured on MI355X, 8 waves per head instead
// of 4 were slower at batch 1-16 (B=1 ctx 512: 15.6 vs 12.9 us, B=8 ctx 512:
// 18.0 vs 14.4 us) and equal on long contexts: these launches are bound by
// latency chains and the cross-wave merge, not by the loads in flight.

// The list workgroup w that hardware workgroup i runs, in KV-head pairs.
// Workgroups are dealt to the XCDs round robin (i % 8). When each pair unit
// is cut into m >= 2 segments (m = grid / list units, a power of two dividing
// the grid here), list order would put a sequence's pairs at the same offset
// (the workgroups reading the same pages at the same time) on one XCD, and
// every XCD would serve all pairs. The transposed order w = (i % rows) * m +
// i / rows (rows = grid / m) makes consecutive i the consecutive pair units
// at one offset, so XCD x serves pair x % 4 of 8 KV heads, as one workgroup
// per unit does: measured at 32/8/128 B=8 ctx 32768 (per-workgroup clock
// stamps), workgroups with equal work end within 155-162 us instead of
// 138-169 us, and the kernel takes 172-177 instead of 178-179 us. Unpaired
// balanced launches keep list order (the same order measured within 1 %).
__device__ __forceinline__ int paired_list_wg(const DecodeArgs& a, int units_per_seq) {
  const int i = static_cast<int>(blockIdx.x);
  const int64_t list_units = static_cast<int64_t>(a.batch) * units_per_seq;
  const int64_t q = list_units > 0 ? a.grid / list_units : 0;
  if (q < 2) return i;
  const int m = 1 << (31 - __builtin_clz(static_cast<unsigned>(q)));
  if (a.grid % m != 0) return i;
  const int rows = a.grid / m;
  return (i % rows) * m + i / rows;
}

// The unit of list unit ui (hp list units per sequence; KV heads PAIR * j +
// half for list unit j of a sequence's hp), wave-uniform.
template <int PAIR>
__device__ __forceinline__ Unit list_unit(const DecodeArgs& a, int hp, int ui, int half) {
  const int b = ui / hp;
  const int r = ui - b * hp;
  const int rkv = a.head_groups == 1 ? r : r / a.head_groups;
  Unit u;
  u.b = __builtin_amdgcn_readfirstlane(b);
  u.kvh = __builtin_amdgcn_readfirstlane(rkv * PAIR + half);
  u.hg = __builtin_amdgcn_readfirstlane(r - rkv * a.head_groups);
  u.split = 0;
  return u;
}

// PAIR = 2 (num_kv_heads even): the work list's units are KV-head pairs (j,
// head group); the workgroup has two halves of W waves that walk the same
// segments, half h streaming KV head 2j + h with its own LDS (adjacent bytes
// of every token row, as in decode_mfma_paired_kernel). Half h of segment
// (list workgroup w, list unit u) owns partial slot (w + u) * 2 + h.
template <typename E, typename KVF, int D, int NT, int PAIR>
__global__ void __launch_bounds__(PAIR * kThreads, (mfma_waves_per_eu<D, NT>()))
    decode_mfma_balanced_kernel(const DecodeArgs a) {
  constexpr int W = kWaves;
  using Lds = MfmaLds<D, NT, W, dma_staged<KVF, D, NT>()>;
  __shared__ __attribute__((aligned(16))) char lds[PAIR * Lds::kBytes];
  __shared__ int s_last[PAIR];
  fetch_args(a);
  // A compile-time 0 with PAIR == 1, so the LDS base stays a constant.
  const int half = PAIR == 2 ? wave_id() / W : 0;
  const int hp = a.num_kv_heads * a.head_groups / PAIR;  // list units per sequence
  const int w = PAIR == 2 ? paired_list_wg(a, hp) : static_cast<int>(blockIdx.x);
  const int hw = wave_id() - half * W;  // wave within the half
  // Even-batch start. When the grid is one workgroup per list unit
  // (even_start) and every sequence has the same page count n >=
  // kMinPagesPerBalancedWg, workgroup w's range is exactly list unit w,
  // whole: the uniform cut. For that case the unit's first block-table
  // window, then seq_lens, then its q are issued before any of them is
  // waited for, as the uniform kernels issue theirs, and the scan is
  // skipped; any other batch runs the schedule below, after the guessed
  // loads land. The order is measured: with q issued before the window
  // (the uniform kernels' order), the whole kernel ran 12-16 % slower on
  // MI355X (32/8/128 fp16 B=64 ctx 4096 187 vs 162 us, ragged 228 vs 205),
  // on the guessed path and on the scan after a failed guess alike, though
  // the main loops compiled to the same instructions; q after the window
  // and seq_lens costs nothing measurable.
  Unit gu{};
  QFrag<NT, D / 32> gq;
  if (a.even_start) {
    gu = list_unit<PAIR>(a, hp, w, half);
    prefetch_window<KVF, D, NT>(a, lds + half * Lds::kBytes, gu.b, 0, a.max_pages, hw);
  }
  LenChunks lc;
  if (a.batch <= 64 * kScanChunks) lc = load_len_chunks(a);
  if (a.even_start) {
    load_q<E, D, NT>(a, gu, gq);
    const int n = even_pages(a, lc);
    if (n >= kMinPagesPerBalancedWg) {
      gu.seq_len = __builtin_amdgcn_readfirstlane(chunk_len(a, lc, gu.b));
      gu.page_begin = 0;
      gu.page_end = n;
      Dest dst{};
      dst.final = true;
      mfma_segment<E, KVF, D, NT, W>(a, lds + half * Lds::kBytes, gu, dst, hw, &gq, true);
      return;
    }
    wait_vmcnt<0>();  // the guessed window loads write LDS the segments below reuse
  }
  const Start st = schedule_start(a, hp, w, lc);
  if (a.arrivals != nullptr) {
    // No merge kernel follows: empty sequences get their zeros here, sequence
    // b from workgroup b % grid (up to 64 * kScanChunks from the schedule's scan).
    auto zero = [&](int b) {
      typename E::S* out = static_cast<typename E::S*>(a.out) + static_cast<int64_t>(b) * a.num_q_heads * D;
      for (int i = threadIdx.x; i < a.num_q_heads * D; i += blockDim.x) out[i] = E::from_f32(0.0f);
    };
    if (a.batch <= 64 * kScanChunks) {
#pragma unroll
      for (int k = 0; k < kScanChunks; ++k) {
        for (uint64_t m = st.empties[k]; m != 0; m &= m - 1) zero(64 * k + __builtin_ctzll(m));
      }
    } else {
      for (int b = blockIdx.x; b < a.batch; b += gridDim.x) {
        if (seq_pages_uniform(a, b) == 0) zero(b);
      }
    }
  }
  int64_t pos = st.pos;
  const int64_t end = min(pos + st.per, st.total);
  int b = st.b;
  int64_t base = st.base;
  int n = st.pages;   // pages of sequence b
  int len = st.len;   // its clamped length
  const int charge = st.charge;

  while (pos < end && b < a.batch) {
    // b is pages-bearing: the start and the advance below skip empty sequences.
    // The offset inside sequence b's units is below hp * (max_pages + charge),
    // so 32-bit arithmetic splits it into a unit and a position (a 64-bit
    // division here, scalar and in software, cost ~0.5 us before every
    // segment's first load). A unit spans charge + n list positions, its
    // pages after the charge (list_prefix).
    const int span = n + charge;
    const uint32_t off = static_cast<uint32_t>(pos - base);
    const uint32_t ru = off / static_cast<uint32_t>(span);
    const int r = static_cast<int>(ru);
    const int at = static_cast<int>(off - ru * static_cast<uint32_t>(span));
    const int64_t unit_base = base + static_cast<int64_t>(r) * span;
    const int64_t page_base = unit_base + charge;  // list position of the unit's page 0
    const int page0 = max(0, at - charge);
    // At most page0 only when the range ends inside the unit's charge: no pages here.
    const int page1 = static_cast<int>(min(static_cast<int64_t>(n), end - page_base));
    if (page1 > page0) {
      // The unit is wave-uniform, but the compiler cannot prove it through the
      // scan above; without readfirstlane the buffer descriptors built from it
      // land in VGPRs and every K/V load becomes a per-lane waterfall loop.
      Unit u;
      u.b = __builtin_amdgcn_readfirstlane(b);
      const int rkv = a.head_groups == 1 ? r : r / a.head_groups;  // one head group is the common case
      u.kvh = __builtin_amdgcn_readfirstlane(rkv * PAIR + half);
      u.hg = __builtin_amdgcn_readfirstlane(r - rkv * a.head_groups);
      u.split = 0;
      u.seq_len = __builtin_amdgcn_readfirstlane(len);
      u.page_begin = __builtin_amdgcn_readfirstlane(page0);
      u.page_end = __builtin_amdgcn_readfirstlane(page1);

      const int64_t slot = (static_cast<int64_t>(w) + static_cast<int64_t>(b) * hp + r) * PAIR + half;
      Dest dst;
      dst.final = page0 == 0 && page1 == n;
      dst.o = a.o_part + slot * a.heads_per_wg * D;
      dst.lse = a.lse_part + slot * a.heads_per_wg;
      dst.o_head_stride = D;
      dst.lse_head_stride = 1;

      // The previous segment's waves may still read LDS; before the first
      // segment nothing has used it (the schedule needs no LDS), so no barrier.
      if (pos != st.pos) __syncthreads();
      mfma_segment<E, KVF, D, NT, W>(a, lds + half * Lds::kBytes, u, dst, hw);
      if (NT == 1 && !dst.final && a.arrivals != nullptr) {  // see kFusedMergeMaxHeads
        // The unit's segments are workgroups w0 .. w1, those whose ranges hold
        // its first and last page (slots (w + list unit) * PAIR + half).
        const int64_t w0 = page_base / st.per;
        const int64_t w1 = (page_base + n - 1) / st.per;
        const int64_t slot0 = (w0 + static_cast<int64_t>(b) * hp + r) * PAIR + half;
        const int h0 = u.hg * a.heads_per_wg;
        MergeJob job;
        job.lse = a.lse_part + slot0 * a.heads_per_wg;
        job.lse_head_stride = 1;
        job.l_stride = static_cast<int64_t>(PAIR) * a.heads_per_wg;
        job.o = a.o_part + slot0 * a.heads_per_wg * D;
        job.o_head_stride = D;
        job.o_stride = static_cast<int64_t>(PAIR) * a.heads_per_wg * D;
        job.n = static_cast<int>(w1 - w0) + 1;
        job.heads = min(a.heads_per_wg, a.group - h0);
        job.out = static_cast<typename E::S*>(a.out) +
                  (static_cast<int64_t>(u.b) * a.num_q_heads + u.kvh * a.group + h0) * D;
        const int64_t unit = (static_cast<int64_t>(u.b) * a.num_kv_heads + u.kvh) * a.head_groups + u.hg;
        arrive_and_merge<E, W>(a.arrivals + unit, job, D, hw, s_last + half);
      }
    }

    pos = page_base + page1;  // end, or the next unit's first list position
    if (pos < end && r == hp - 1 && page1 == n) {  // more to do past this sequence: next non-empty one
      base += static_cast<int64_t>(span) * hp;
      do {
        b = __builtin_amdgcn_readfirstlane(b + 1);
        len = b < a.batch ? clamped_len(a, as_constant(a.seq_lens)[b]) : 0;
        n = pages_of(a, len);
      } while (b < a.batch && n == 0);
    }
  }
}

// ------------------------------------------------------------ VALU split path

// The elements of a 16-byte slice as floats. The fp32 case bit-casts the whole
// vector: this compiler lowers __builtin_bit_cast of a single vector element
// (`bit_cast<float>(v[i])`) to element 0 for every i.
template <typename E>
__device__ __forceinline__ void unpack16(u32x4 v, float (&f)[16 / E::kBytes]) {
  if constexpr (E::kBytes == 4) {
    const f32x4 fv = __builtin_bit_cast(f32x4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = fv[i];
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = lo_f32<E>(v[i]);
      f[2 * i + 1] = hi_f32<E>(v[i]);
    }
  }
}

template <int TPT>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int mask = 1; mask < TPT; mask <<= 1) v += shfl_xor(v, mask);
  return v;
}

template <typename E, int D, int GMAX>
struct ValuCfg {
  static constexpr int kVec = 16 / E::kBytes;                     // elements per 16-byte slice
  static constexpr int kTpt = D / kVec;                           // lanes per token
  static constexpr int kTpw = 64 / kTpt;                          // tokens per wave step
  static constexpr int kLdsFloats = kWaves * GMAX * (D + 2);
};

template <typename E, int D, int GMAX>
__global__ void __launch_bounds__(kThreads) decode_valu_kernel(const DecodeArgs a) {
  using S = typename E::S;
  using C = ValuCfg<E, D, GMAX>;
  constexpr int VEC = C::kVec;
  constexpr int TPT = C::kTpt;
  constexpr int TPW = C::kTpw;
  static_assert(TPT >= 1 && TPT <= 64 && (TPT & (TPT - 1)) == 0, "head_dim slices must tile a wave");
  __shared__ float lds[C::kLdsFloats];

  const Unit u = decode_unit(a);
  if (u.page_begin >= u.page_end) {
    if (u.split == 0 && u.seq_len <= 0 && a.num_splits == 1) {
      write_zero_heads<typename E::S, E>(a, u, D, threadIdx.x, blockDim.x);
    }
    return;
  }
  const int lane = __lane_id();
  const int wave = wave_id();
  const int slot = lane / TPT;
  const int dv = (lane % TPT) * VEC;
  const int h0 = u.hg * a.heads_per_wg;
  const int nh = min(GMAX, a.group - h0);

  float qv[GMAX][VEC];
  {
    const S* q = static_cast<const S*>(a.q);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      const int hl = g < nh ? h0 + g : h0;
      const S* qh = q + (static_cast<int64_t>(u.b) * a.num_q_heads + u.kvh * a.group + hl) * D + dv;
#pragma unroll
      for (int e = 0; e < VEC; ++e) qv[g][e] = g < nh ? E::to_f32(qh[e]) : 0.0f;
    }
  }

  float m[GMAX], l[GMAX], acc[GMAX][VEC];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[g][e] = 0.0f;
  }

  const S* kc = static_cast<const S*>(a.k);
  const S* vc = static_cast<const S*>(a.v);
  const int32_t* bt = a.block_table + static_cast<int64_t>(u.b) * a.bt_stride;
  const int tok_begin = u.page_begin * a.page_size;
  const int tok_end = min(u.page_end * a.page_size, u.seq_len);
  const int steps = (tok_end - tok_begin + kWaves * TPW - 1) / (kWaves * TPW);

  for (int it = 0; it < steps; ++it) {
    const int tok = tok_begin + it * kWaves * TPW + wave * TPW + slot;
    const bool valid = tok < tok_end;
    u32x4 kx = {0, 0, 0, 0}, vx = {0, 0, 0, 0};
    if (valid) {
      const int64_t page = bt[tok / a.page_size];
      const int64_t off = page * a.page_stride + static_cast<int64_t>(tok % a.page_size) * a.token_stride +
                          static_cast<int64_t>(u.kvh) * D + dv;
      kx = *reinterpret_cast<const u32x4*>(kc + off);
      vx = *reinterpret_cast<const u32x4*>(vc + off);
    }
    float kf[VEC], vf[VEC];
    unpack16<E>(kx, kf);
    unpack16<E>(vx, vf);
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      float dot = 0.0f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) dot += qv[g][e] * kf[e];
      const float s = group_sum<TPT>(dot) * a.scale_log2;
      if (valid) {
        const float m_new = fmaxf(m[g], s);
        const float alpha = exp2f(m[g] - m_new);
        const float p = exp2f(s - m_new);
        l[g] = l[g] * alpha + p;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[g][e] = acc[g][e] * alpha + p * vf[e];
        m[g] = m_new;
      }
    }
  }

  // Merge the token slots of this wave (lanes with equal dims), log-sum-exp rule.
#pragma unroll
  for (int mask = TPT; mask < 64; mask <<= 1) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      const float mo = shfl_xor(m[g], mask);
      const float lo = shfl_xor(l[g], mask);
      const float mm = fmaxf(m[g], mo);
      const float c0 = m[g] == -INFINITY ? 0.0f : exp2f(m[g] - mm);
      const float c1 = mo == -INFINITY ? 0.0f : exp2f(mo - mm);
      l[g] = l[g] * c0 + lo * c1;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float ao = shfl_xor(acc[g][e], mask);
        acc[g][e] = acc[g][e] * c0 + ao * c1;
      }
      m[g] = mm;
    }
  }

  // Merge the waves through LDS; wave 0 writes.
  float* wl = lds + wave * GMAX * (D + 2);
  if (slot == 0) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) wl[g * (D + 2) + dv + e] = acc[g][e];
      if (dv == 0) {
        wl[g * (D + 2) + D] = m[g];
        wl[g * (D + 2) + D + 1] = l[g];
      }
    }
  }
  __syncthreads();
  if (wave != 0 || slot != 0) return;
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= nh) break;
    float mw[kWaves], mmax = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      mw[w] = lds[(w * GMAX + g) * (D + 2) + D];
      mmax = fmaxf(mmax, mw[w]);
    }
    float cw[kWaves], denom = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      cw[w] = mw[w] == -INFINITY ? 0.0f : exp2f(mw[w] - mmax);
      denom += lds[(w * GMAX + g) * (D + 2) + D + 1] * cw[w];
    }
    const int64_t head = static_cast<int64_t>(u.b) * a.num_q_heads + u.kvh * a.group + h0 + g;
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float num = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) num += lds[(w * GMAX + g) * (D + 2) + dv + e] * cw[w];
      const float o = num / denom;
      if (a.num_splits == 1) {
        static_cast<S*>(a.out)[head * D + dv + e] = E::from_f32(o);
      } else {
        a.o_part[(head * a.num_splits + u.split) * D + dv + e] = o;
      }
    }
    if (a.num_splits > 1 && dv == 0) a.lse_part[head * a.num_splits + u.split] = mmax + log2f(denom);
  }
}

// --------------------------------------------------------------- split merge

// Merge of n partials (o_w, lse_w), w = 0 .. n-1, into one output head, by
// one wave: out[d] = sum_w 2^(lse_w - M) o_w[d] / sum_w 2^(lse_w - M),
// M = max_w lse_w. o_w[d] is at op[w * o_stride + d] (16-byte aligned rows),
// lse_w at lse[w * l_stride]; head_dim is a power of two from 16 to 256.
//
// Lane l reads 16 bytes (dims 4c .. 4c+3, c = l mod C, C = head_dim / 4) of
// partial rows l / C, l / C + R, ... (R = 64 / C rows per wave-wide load),
// up to kG rows per lane per round, each with its lse. The first round's loads go
// out before the lse loads of the max and the sum, so for up to kG * R
// partials (32 at head_dim 128 with kG = 16) the merge waits for memory once.
// Indexes are clamped (weight 0 past the end); rows are then summed across the
// R lane groups with xor shuffles. Each lane group adds its rows in increasing
// order whatever kG is, so every kG gives the same bits.
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  return fmaxf(fmaxf(lane_read(v, 0), lane_read(v, 16)), fmaxf(lane_read(v, 32), lane_read(v, 48)));
}

template <typename E, int kG, int POL>
__device__ __forceinline__ void merge_partials(const float* lse, int64_t l_stride, const float* op,
                                               int64_t o_stride, int n, int head_dim, typename E::S* out) {
  const int lane = __lane_id();
  const int cpr = head_dim >> 2;      // 16-byte chunks per row (4 .. 64)
  const int rpl = 64 / cpr;           // rows per wave-wide load
  const int c = lane & (cpr - 1);
  const int r = lane / cpr;
  // POL != 0: buffer loads with that cache policy (op and lse are
  // wave-uniform, a unit's partials lie within 2 GiB of them).
  const auto orsrc = make_rsrc(uniform_ptr(op));
  const auto lrsrc = make_rsrc(uniform_ptr(lse));
  auto load_o = [&](int w) -> f32x4 {
    if constexpr (POL == 0) {
      return *reinterpret_cast<const f32x4*>(op + w * o_stride + 4 * c);
    } else {
      return __builtin_bit_cast(f32x4, buffer_load16<POL>(orsrc, static_cast<uint32_t>((w * o_stride + 4 * c) * 4)));
    }
  };
  auto load_lse = [&](int w) -> float {
    if constexpr (POL == 0) {
      return lse[w * l_stride];
    } else {
      return buffer_load_f32<POL>(lrsrc, static_cast<uint32_t>(w * l_stride * 4));
    }
  };
  f32x4 v[kG];
  float lw[kG];
  auto load_round = [&](int base) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      lw[j] = -INFINITY;
      if (base + rpl * j < n) {  // wave-uniform: some lane has a row here
        const int w = min(base + r + rpl * j, n - 1);
        v[j] = load_o(w);
        lw[j] = load_lse(w);
      }
    }
  };
  load_round(0);
  float mx = -INFINITY;
  for (int w = lane; w < n; w += 64) mx = fmaxf(mx, load_lse(w));
  mx = wave_max(mx);
  float den = 0.0f;
  for (int w = lane; w < n; w += 64) den += exp2f(load_lse(w) - mx);
  den = wave_sum(den);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int per_round = kG * rpl;
  for (int base = 0; base < n; base += per_round) {
    if (base > 0) load_round(base);
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const float wt = base + r + rpl * j < n ? exp2f(lw[j] - mx) : 0.0f;
      acc += wt * v[j];
    }
  }
  for (int off = cpr; off < 64; off <<= 1) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += __shfl_xor(acc[k], off, 64);
  }
  if (r == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[4 * c + k] = E::from_f32(acc[k] / den);
  }
}

// merge_partials split into a load phase and a finish phase, for merges whose
// rows all fit one round (n <= kG * 256 / head_dim) and n <= 64, so a wave can
// issue the next head's loads before it finishes this one. The arithmetic is
// merge_partials' own: with n <= 64, its max and sum loops give lane l the lse
// of row l (or -inf / 0 past n), which `ll` holds here; rows past n weigh 0.
// The results are therefore bit-identical to merge_partials.
template <int kG, int POL>
__device__ __forceinline__ void head_merge_load(HeadMerge<kG>& m, const float* lse, int64_t l_stride, const float* op,
                                                int64_t o_stride, int n, int head_dim) {
  const int lane = __lane_id();
  const int cpr = head_dim >> 2;
  const int rpl = 64 / cpr;
  const int c = lane & (cpr - 1);
  const int r = lane / cpr;
  const auto orsrc = make_rsrc(uniform_ptr(op));
  const auto lrsrc = make_rsrc(uniform_ptr(lse));
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    m.v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    m.lw[j] = -INFINITY;
    if (rpl * j < n) {
      const int w = min(r + rpl * j, n - 1);
      m.v[j] = __builtin_bit_cast(f32x4, buffer_load16<POL>(orsrc, static_cast<uint32_t>((w * o_stride + 4 * c) * 4)));
      m.lw[j] = buffer_load_f32<POL>(lrsrc, static_cast<uint32_t>(w * l_stride * 4));
    }
  }
  m.ll = lane < n ? buffer_load_f32<POL>(lrsrc, static_cast<uint32_t>(lane * l_stride * 4)) : -INFINITY;
}

template <typename E, int kG>
__device__ __forceinline__ void head_merge_finish(const HeadMerge<kG>& m, int n, int head_dim, typename E::S* out) {
  const int lane = __lane_id();
  const int cpr = head_dim >> 2;
  const int rpl = 64 / cpr;
  const int c = lane & (cpr - 1);
  const int r = lane / cpr;
  const float mx = wave_max(m.ll);
  const float den = wave_sum(lane < n ? exp2f(m.ll - mx) : 0.0f);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < kG; ++j) {
    const float wt = r + rpl * j < n ? exp2f(m.lw[j] - mx) : 0.0f;
    acc += wt * m.v[j];
  }
  for (int off = cpr; off < 64; off <<= 1) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] += __shfl_xor(acc[k], off, 64);
  }
  if (r == 0) {
#pragma unroll
    for (int k = 0; k < 4; ++k) out[4 * c + k] = E::from_f32(acc[k] / den);
  }
}

// out[b, h] = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M) over the splits that
// hold tokens of sequence b (kernel_lab/triton_kernels/paged_attention.py:134-166).
// Splits past the end of a sequence are never read, so their workspace may hold
// anything.
template <typename E>
__global__ void __launch_bounds__(64) decode_merge_kernel(const DecodeArgs a, int head_dim) {
  using S = typename E::S;
  const int bh = blockIdx.x;
  const int b = bh / a.num_q_heads;
  const int lane = __lane_id();
  const int raw = a.seq_lens[b];
  const int64_t cap = static_cast<int64_t>(a.max_pages) * a.page_size;
  const int seq_len = static_cast<int>(raw < cap ? raw : cap);
  const int num_pages = seq_len > 0 ? (seq_len + a.page_size - 1) / a.page_size : 0;
  const int active = min(a.num_splits, (num_pages + a.pages_per_split - 1) / a.pages_per_split);
  S* out = static_cast<S*>(a.out) + static_cast<int64_t>(bh) * head_dim;
  if (active <= 0) {
    for (int d = lane; d < head_dim; d += 64) out[d] = E::from_f32(0.0f);
    return;
  }
  const float* lse = a.lse_part + static_cast<int64_t>(bh) * a.num_splits;
  const float* op = a.o_part + static_cast<int64_t>(bh) * a.num_splits * head_dim;
  merge_partials<E>(lse, 1, op, head_dim, active, head_dim, out);
}

// Merge for the balanced schedule: one wave per (sequence, query head). Units
// that one workgroup covered were written by the decode kernel; a unit spread
// over workgroups w0..w1 is combined from slots w + unit by the LSE rule; an
// empty sequence (no units) gets zeros here.
template <typename E>
__global__ void __launch_bounds__(64) decode_merge_balanced_kernel(const DecodeArgs a, int head_dim) {
  using S = typename E::S;
  const int lane = __lane_id();
  const int b = blockIdx.x / a.num_q_heads;
  const int head = blockIdx.x % a.num_q_heads;
  const int kvh = head / a.group;
  const int hl = head % a.group;
  const int hg = hl / a.heads_per_wg;
  const int hloc = hl % a.heads_per_wg;
  const int pair = a.paired ? 2 : 1;  // list units are KV-head pairs (decode_mfma_balanced_kernel<..., 2>)
  const int hp = a.num_kv_heads * a.head_groups / pair;
  int64_t total, base;  // list length; list position of sequence b's first unit
  int n, charge;        // sequence b's pages; list positions ahead of each unit's pages
  list_prefix(a, hp, b, &total, &base, &n, &charge);
  S* out = static_cast<S*>(a.out) + (static_cast<int64_t>(b) * a.num_q_heads + head) * head_dim;
  if (n == 0) {
    // No cached token: the softmax-weighted sum over no values is zero.
    for (int d = lane; d < head_dim; d += 64) out[d] = E::from_f32(0.0f);
    return;
  }
  const int64_t per = balanced_per(a, total);
  const int r = (kvh / pair) * a.head_groups + hg;
  const int64_t page_base = base + static_cast<int64_t>(r) * (n + charge) + charge;  // the unit's page 0
  const int64_t w0 = page_base / per;
  const int64_t w1 = (page_base + n - 1) / per;
  if (w0 == w1) return;
  const int64_t uidx = static_cast<int64_t>(b) * hp + r;
  const int64_t slot0 = (w0 + uidx) * pair + kvh % pair;  // consecutive workgroups' slots are `pair` apart
  const float* lse = a.lse_part + hloc;
  const float* op = a.o_part + static_cast<int64_t>(hloc) * head_dim;
  const int64_t stride_l = a.heads_per_wg;
  const int64_t stride_o = static_cast<int64_t>(a.heads_per_wg) * head_dim;

  const int nw = static_cast<int>(w1 - w0) + 1;
  merge_partials<E>(lse + slot0 * stride_l, pair * stride_l, op + slot0 * stride_o, pair * stride_o, nw, head_dim,
                    out);
}

// ---------------------------------------------------- cascade (shared prefix)
//
// Cascade decode: every sequence attends over a shared prefix (one block-table
// row of prefix_len tokens) followed by its own tokens. The prefix pass runs
// the MFMA segment with all sequences' query heads of a KV head folded into
// one group (q_fold), so each workgroup streams the prefix once for up to 32
// query rows of many sequences; the suffix pass is the plain split decode.
// Both write fp32 partials, and this kernel merges them by the LSE rule.

struct CascadeArgs {
  const float* p_o;          // prefix partials: virtual head kvh*(B*G) + b*G + g, p_splits each
  const float* p_lse;
  const int32_t* prefix_len; // device, one value
  int prefix_pages;          // prefix block-table length
  int p_splits, p_pps;
  const float* s_o;          // suffix partials: head b*Hq + h, s_splits each
  const float* s_lse;
  const int32_t* seq_lens;
  int max_pages;
  int s_splits, s_pps;
  void* out;
  int batch, num_q_heads, group, page_size;
};

// Splits of a pass that hold tokens of a sequence of `len` tokens.
__device__ __forceinline__ int active_splits(int len, int max_pages, int page_size, int splits, int pps) {
  const int64_t cap = static_cast<int64_t>(max_pages) * page_size;
  const int n = static_cast<int>(len < cap ? len : cap);
  const int pages = n > 0 ? (n + page_size - 1) / page_size : 0;
  return min(splits, (pages + pps - 1) / pps);
}

// Adds n partials (o_w at o + w*D, lse_w at lse[w]) to a running
// sum_w 2^(lse_w - mx) o_w[d], loads issued eight partials at a time.
__device__ __forceinline__ float merge_accumulate(const float* lse, const float* o, int n, int head_dim, int d,
                                                  float mx) {
  constexpr int U = 8;
  float num = 0.0f;
  for (int w0 = 0; w0 < n; w0 += U) {
    float wt[U], v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
      const int w = min(w0 + j, n - 1);
      wt[j] = lse[w];
      v[j] = o[static_cast<int64_t>(w) * head_dim + d];
    }
#pragma unroll
    for (int j = 0; j < U; ++j) num += (w0 + j < n ? exp2f(wt[j] - mx) : 0.0f) * v[j];
  }
  return num;
}

template <typename E>
__global__ void __launch_bounds__(64) cascade_merge_kernel(const CascadeArgs c, int head_dim) {
  using S = typename E::S;
  const int lane = __lane_id();
  const int b = blockIdx.x / c.num_q_heads;
  const int h = blockIdx.x % c.num_q_heads;
  const int kvh = h / c.group;
  const int g = h % c.group;
  const int np = active_splits(as_constant(c.prefix_len)[0], c.prefix_pages, c.page_size, c.p_splits, c.p_pps);
  const int ns = active_splits(as_constant(c.seq_lens)[b], c.max_pages, c.page_size, c.s_splits, c.s_pps);
  const int64_t shead = static_cast<int64_t>(b) * c.num_q_heads + h;
  S* out = static_cast<S*>(c.out) + shead * head_dim;
  if (np + ns == 0) {
    for (int d = lane; d < head_dim; d += 64) out[d] = E::from_f32(0.0f);
    return;
  }
  const int64_t vhead = (static_cast<int64_t>(kvh) * c.batch + b) * c.group + g;
  const float* pl = c.p_lse + vhead * c.p_splits;
  const float* po = c.p_o + vhead * c.p_splits * head_dim;
  const float* sl = c.s_lse + shead * c.s_splits;
  const float* so = c.s_o + shead * c.s_splits * head_dim;
  float mx = -INFINITY;
  for (int w = lane; w < np; w += 64) mx = fmaxf(mx, pl[w]);
  for (int w = lane; w < ns; w += 64) mx = fmaxf(mx, sl[w]);
  mx = wave_max(mx);
  float den = 0.0f;
  for (int w = lane; w < np; w += 64) den += exp2f(pl[w] - mx);
  for (int w = lane; w < ns; w += 64) den += exp2f(sl[w] - mx);
  den = wave_sum(den);
  for (int d = lane; d < head_dim; d += 64) {
    const float num = merge_accumulate(pl, po, np, head_dim, d, mx) + merge_accumulate(sl, so, ns, head_dim, d, mx);
    out[d] = E::from_f32(num / den);
  }
}

// -------------------------------------------------------------- host side

// Sets the page size and the multiplier / shift of the block -> page
// division (block_page). With d = blocks per page, l = ceil(log2 d) and
// p = 31 + l, m = ceil(2^p / d) is below 2^32, and for 0 <= n < 2^31
// n m / 2^p = n / d + n e / (d 2^p) with e = m d - 2^p in [0, d): the excess
// is below 2^31 / 2^p = 2^-l <= 1 / d, so the floor is floor(n / d).
void set_page_size(DecodeArgs& a, int page_size) {
  a.page_size = page_size;
  const uint64_t d = static_cast<uint64_t>(std::max(1, page_size / kBlock));
  int l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  a.bpp_shift = 31 + l;
  a.bpp_magic = static_cast<uint32_t>(((uint64_t{1} << a.bpp_shift) + d - 1) / d);
}

// Shapes the MFMA kernels serve.
bool mfma_path(kl_dtype dtype, int head_dim, int page_size) {
  return (dtype == KL_DTYPE_F16 || dtype == KL_DTYPE_BF16) && page_size % kBlock == 0 &&
         (head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256);
}

// Switches for A/B measurements and tests; unset, the library behaves as
// planned below. They are read from the environment once per process, at
// the first call that needs them, and again by
// kl_paged_decode_reload_options():
//   KL_DECODE_FORCE_VALU=1        16-bit decode on the VALU kernel, so the
//                                 benchmarks can time both paths on the same
//                                 shapes (the FP8 and cascade entry points
//                                 ignore it)
//   KL_DECODE_PAIRED=0            no paired (two KV heads) workgroups
//   KL_DECODE_BALANCE_ALWAYS=1|0  full batches always balanced | always
//                                 uniform (the default chooses by table
//                                 length; see make_plan)
//   KL_DECODE_FUSED_MERGE=0       split decodes merge in a separate launch
struct Options {
  static constexpr unsigned kLoaded = 1, kForceValu = 2, kNoPairs = 4, kNoFusedMerge = 8, kBalanceAlways = 16,
                            kBalanceNever = 32;
  unsigned bits = kLoaded;
  bool force_valu() const { return (bits & kForceValu) != 0; }
  bool pairing() const { return (bits & kNoPairs) == 0; }
  bool fused_merge() const { return (bits & kNoFusedMerge) == 0; }
  // Full-batch schedule: 1 balanced, 0 uniform, -1 by table length.
  int balance() const { return (bits & kBalanceAlways) ? 1 : (bits & kBalanceNever) ? 0 : -1; }
};

std::atomic<unsigned> g_option_bits{0};  // 0: not read yet

unsigned read_option_bits() {
  auto starts = [](const char* name, char c) {
    const char* v = std::getenv(name);
    return v != nullptr && v[0] == c;
  };
  unsigned bits = Options::kLoaded;
  if (starts("KL_DECODE_FORCE_VALU", '1')) bits |= Options::kForceValu;
  if (starts("KL_DECODE_PAIRED", '0')) bits |= Options::kNoPairs;
  if (starts("KL_DECODE_FUSED_MERGE", '0')) bits |= Options::kNoFusedMerge;
  if (starts("KL_DECODE_BALANCE_ALWAYS", '1')) bits |= Options::kBalanceAlways;
  if (starts("KL_DECODE_BALANCE_ALWAYS", '0')) bits |= Options::kBalanceNever;
  return bits;
}

Options options() {
  Options o;
  o.bits = g_option_bits.load(std::memory_order_relaxed);
  if (o.bits == 0) {
    o.bits = read_option_bits();
    g_option_bits.store(o.bits, std::memory_order_relaxed);
  }
  return o;
}

// Device address of a file-scope __device__ array on the current device.
// The lookup is not a stream operation, but the first one may load the code
// object, a call the runtime can refuse while any thread captures a graph in
// the global mode (torch.cuda.graph's default); this thread's capture mode is
// relaxed for the lookup and restored after it.
template <typename T>
hipError_t device_symbol_address(void** p, const T& symbol) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
  const hipError_t err = hipGetSymbolAddress(p, reinterpret_cast<const void*>(&symbol));
  if (swapped) {
    (void)hipThreadExchangeStreamCaptureMode(&mode);
  } else {
    (void)hipGetLastError();  // the failed exchange must not reach the launch check
  }
  return err;
}

// The arrival-counter region for a fused call on `stream` (current device),
// or null for the merge kernel.
//   eager stream      the stream's own region, taken on its first fused call
//                     and kept (its calls run one after another);
//   capturing stream  a region of its own for each (capture sequence, capture
//                     stream): every launch of the resulting graph node
//                     replays with it, and a graph never runs concurrently
//                     with itself, while two graphs, or a graph and eager
//                     work, may; regions of captures are never reused (the
//                     library cannot see a graph's destruction);
//   hipStreamPerThread, a broken capture, or an unreadable stream: none.
// A pool that runs out is reported once per device on stderr.
uint32_t* arrival_region(hipStream_t stream) {
  if (stream == hipStreamPerThread) return nullptr;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  unsigned long long capture = 0;
  if (hipStreamGetCaptureInfo(stream, &cs, &capture) != hipSuccess) {
    (void)hipGetLastError();  // the launch check must not see this error
    return nullptr;
  }
  if (cs == hipStreamCaptureStatusInvalidated) return nullptr;
  const bool capturing = cs == hipStreamCaptureStatusActive;
  struct Owner {
    hipStream_t stream;
    unsigned long long capture;  // 0: eager
  };
  struct Device {
    uint32_t* base = nullptr;
    bool located = false;
    Owner eager[kStreamRegions] = {};
    Owner captured[kCaptureRegions] = {};
    int eager_taken = 0;
    int captured_taken = 0;
    bool warned_eager = false;
    bool warned_captured = false;
  };
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static Device devices[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  const unsigned long long key = capturing ? capture : 0;
  // Most calls repeat the calling thread's last (device, stream, capture):
  // regions are never handed back, so its answer still holds.
  struct Last {
    int dev = -1;
    hipStream_t stream = nullptr;
    unsigned long long key = 0;
    bool capturing = false;
    uint32_t* region = nullptr;
  };
  thread_local Last last;
  if (last.region != nullptr && last.dev == dev && last.stream == stream && last.key == key &&
      last.capturing == capturing) {
    return last.region;
  }
  std::lock_guard<std::mutex> lock(mu);
  Device& d = devices[dev];
  if (!d.located) {
    d.located = true;
    void* p = nullptr;
    // The device array's own name is a host-side stand-in: its device address
    // comes from the runtime, once per device.
    if (device_symbol_address(&p, g_decode_arrivals) == hipSuccess) {
      d.base = static_cast<uint32_t*>(p);
    } else {
      (void)hipGetLastError();  // the merge kernel serves this device; the launch check must not see this error
    }
  }
  if (d.base == nullptr) return nullptr;
  Owner* pool = capturing ? d.captured : d.eager;
  int& taken = capturing ? d.captured_taken : d.eager_taken;
  const int size = capturing ? kCaptureRegions : kStreamRegions;
  const int first = capturing ? kStreamRegions : 0;  // region index of the pool's first entry
  auto remember = [&](int i) {
    last = Last{dev, stream, key, capturing, d.base + static_cast<size_t>(first + i) * kArrivalCounters};
    return last.region;
  };
  for (int i = 0; i < taken; ++i) {
    if (pool[i].stream == stream && pool[i].capture == key) return remember(i);
  }
  if (taken == size) {
    bool& warned = capturing ? d.warned_captured : d.warned_eager;
    if (!warned) {
      warned = true;
      std::fprintf(stderr,
                   "kernel_lab: device %d: all %d split-merge counter regions for %s are taken; further split "
                   "decode calls there use the separate merge kernel (same results, a few microseconds slower)\n",
                   dev, size, capturing ? "graph captures" : "streams");
    }
    return nullptr;
  }
  pool[taken] = Owner{stream, key};
  return remember(taken++);
}

// How the last decode launch on this thread combined split units
// (kl_paged_decode_last_merge).
thread_local int g_last_merge = KL_MERGE_NONE;

// Arrival counters for a split decode of `units` units with up to
// heads_per_wg heads each on the MFMA path, or null for the merge kernel.
uint32_t* fused_merge_counters(const DecodeArgs& a, int64_t units, hipStream_t stream) {
  if (!options().fused_merge() || units > kArrivalCounters || a.heads_per_wg > kFusedMergeMaxHeads) return nullptr;
  if (a.q_fold != a.group || a.force_partial) return nullptr;  // cascade passes keep their own merge
  // Segments per unit: the split count, or for the balanced schedule the
  // workgroups per list unit on even lengths.
  const int64_t list_units = std::max<int64_t>(1, a.grid > 0 && a.paired ? units / 2 : units);
  const int64_t segments = a.grid > 0 ? cdiv(a.grid, list_units) : a.num_splits;
  if (cdiv(a.heads_per_wg, kWaves) * segments > kFusedMergeMaxWork) return nullptr;
  return arrival_region(stream);
}

bool valu_head_dim_ok(kl_dtype dtype, int head_dim) {
  const int vec = dtype == KL_DTYPE_F32 ? 4 : 8;
  switch (head_dim) {
    case 16:
    case 32:
    case 64:
    case 128:
    case 256:
      return head_dim / vec <= 64 && head_dim >= vec;
    default:
      return false;
  }
}

// Query heads one workgroup takes from a GQA group, and the resulting number of
// workgroups per (sequence, KV head, split).
void head_tiling(bool mfma, int head_dim, int group, int* per_wg, int* groups) {
  int cap;
  if (mfma) {
    cap = (group > 16 && head_dim <= 128) ? 32 : 16;
  } else {
    cap = 8;
  }
  int per = std::min(group, cap);
  if (!mfma) {
    per = per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;  // template sizes of the VALU kernel
  }
  *per_wg = per;
  *groups = static_cast<int>(cdiv(group, per));
}

struct Plan {
  int num_splits;       // uniform splits; 0 with the balanced schedule
  int pages_per_split;
  int heads_per_wg;
  int head_groups;
  int grid;             // balanced-schedule workgroups; 0 for uniform splits
  bool paired;          // uniform splits: two adjacent KV heads per 8-wave workgroup
  size_t o_bytes;
  size_t ws_bytes;
};

constexpr size_t kAlign = 256;
size_t align_up(size_t n) { return (n + kAlign - 1) / kAlign * kAlign; }

// partials: a pass of cascade decode, which always takes uniform splits and
// writes fp32 partials (workspace sized for them even with one split).
// use_mfma false: plan for the VALU kernel even where the MFMA one could run.
int make_plan(const Options& opt, kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads, int head_dim,
              int page_size, int max_pages, int num_splits, int cu_count, Plan* p, bool partials = false,
              bool use_mfma = true) {
  if (batch < 0 || num_q_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || page_size <= 0 || max_pages < 0) {
    return fail(KL_ERR_INVALID_ARGUMENT, "batch, heads, head_dim, page_size and max_pages must be positive");
  }
  if (num_q_heads % num_kv_heads != 0) {
    return fail(KL_ERR_INVALID_ARGUMENT, "num_q_heads must be a multiple of num_kv_heads");
  }
  if (num_splits < KL_SPLITS_BALANCED) {
    return fail(KL_ERR_INVALID_ARGUMENT, "num_splits must be >= 0, or KL_SPLITS_BALANCED (-1)");
  }
  if (dtype != KL_DTYPE_F32 && dtype != KL_DTYPE_F16 && dtype != KL_DTYPE_BF16) {
    return fail(KL_ERR_UNSUPPORTED, "dtype must be f32, f16 or bf16");
  }
  const bool mfma = use_mfma && mfma_path(dtype, head_dim, page_size);
  if (!mfma && !valu_head_dim_ok(dtype, head_dim)) {
    return fail(KL_ERR_UNSUPPORTED, "head_dim must be 16, 32, 64, 128 or 256");
  }
  const int group = num_q_heads / num_kv_heads;
  head_tiling(mfma, head_dim, group, &p->heads_per_wg, &p->head_groups);
  const int pages = std::max(max_pages, 1);
  p->grid = 0;
  p->paired = false;
  const int cus = cu_count > 0 ? cu_count : 256;
  const int64_t units = std::max<int64_t>(1, static_cast<int64_t>(batch) * num_kv_heads * p->head_groups);
  if (num_splits == KL_SPLITS_BALANCED && (!mfma || partials)) num_splits = 0;  // uniform splits only
  // The balanced schedule runs in KV-head pairs (8-wave workgroups) on
  // batches that fill the device twice over, as uniform splits would, and on
  // long contexts that give every workgroup half long segments of few-way
  // split pair units (kPairMinPages, kPairMaxSegments).
  const int64_t pair_units = units / 2;
  const bool long_pairs = pair_units * pages >= static_cast<int64_t>(cus) * kPairMinPages &&
                          pair_units * kPairMaxSegments >= cus;
  const bool pairable = mfma && !partials && opt.pairing() && num_kv_heads % 2 == 0 && head_dim <= 128 &&
                        p->heads_per_wg <= 16 && (units >= 2 * static_cast<int64_t>(cus) || long_pairs);
  // Batches whose units fill the device (units >= CUs) take the balanced
  // schedule too. The planner cannot see seq_lens, and with uniform splits
  // one long sequence among short ones sets the time: measured on MI355X
  // (events, us, same tensors alternating), one 65,536-token sequence among
  // 63 of 2,048 tokens 1,231 (uniform) vs 142 (balanced), ragged U[1, 8192]
  // B=64 228 vs 207. A full batch gets one workgroup per list unit, so on an
  // even batch each workgroup's range is one whole unit, the uniform cut,
  // and the kernel starts it as the uniform kernels do (its even-batch
  // start); the choice between the two cuts is made on the device. Where a
  // split unit would need the separate merge launch (more than
  // kFusedMergeMaxHeads query heads per workgroup, or the fused merge
  // switched off), short tables keep uniform splits: that launch costs more
  // than a short table's worst skew.
  const int full_batch_choice = opt.balance();  // 1 balanced, 0 uniform, -1 by default
  const bool full_default =
      (p->heads_per_wg <= kFusedMergeMaxHeads && opt.fused_merge()) || pages >= kBalanceMinPages;
  // The balanced kernel sums 64 sequences' list lengths (their units' pages
  // and charges) in 32-bit lanes and splits a position inside one sequence's
  // units with a 32-bit division; tables long enough to pass 2^31 there keep
  // uniform splits, requested or not.
  const bool list_fits = static_cast<int64_t>(64) * num_kv_heads * p->head_groups *
                             (static_cast<int64_t>(pages) + kMaxSegmentCharge) <= 0x7fffffffLL;
  const bool requested = num_splits == KL_SPLITS_BALANCED && list_fits;
  if (num_splits == KL_SPLITS_BALANCED && !list_fits) num_splits = 0;
  // One sequence cannot be skewed: uniform splits cut it as evenly as the
  // balanced schedule would, without its start (the seq_lens scan before the
  // first block-table load) or its merge's search for each unit's slots.
  // Measured on MI355X (events, us, balanced -> uniform, 32/8/128 fp16 B=1):
  // ctx 512 11.24 -> 9.92, ctx 4096 16.28 -> 13.20, ctx 32768 33.04 -> 31.76;
  // 8/1/128 ctx 32768 26.08 -> 16.40.
  const bool single = batch == 1 && !long_pairs;
  const bool automatic =
      num_splits == 0 && !single && list_fits &&
      (units < cus || (full_batch_choice < 0 ? full_default : full_batch_choice == 1));
  const bool balance = requested || automatic;
  const bool pair_balanced = pairable && balance;
  if (mfma && !partials && balance) {
    // Requested, fewer units than CUs, or a full batch by default: pages
    // balanced across sequences on the device.
    const int64_t lunits = pair_balanced ? units / 2 : units;  // units of the work list
    const int64_t upper = lunits * pages;                        // list length if every sequence were full
    // Paired: one 8-wave workgroup per CU is the register budget, so more
    // workgroups would run in rounds, each paying the schedule's start.
    const int64_t floor_wgs =
        pair_balanced ? static_cast<int64_t>(cus) : std::max<int64_t>(cus, lunits);
    // At most kMaxPlannedSplits workgroups per list unit, as for uniform
    // splits: 8/1/128 fp16 B=2 ctx 32768 took 22.1 us as 256 workgroups (128
    // per sequence) and 17.2 us as 64 uniform splits.
    int64_t grid = std::max<int64_t>(
        1, std::min<int64_t>({cdiv(upper, kMinPagesPerBalancedWg), floor_wgs, lunits * kMaxPlannedSplits, 0x7fffffffLL}));
    // Units merged in the kernel are cut into at most kFusedMaxSegments
    // segments while a full sequence's segments would stay under 32 pages and
    // the cut still gives at least half the CUs a workgroup. Measured on
    // MI355X (events, us, 256 workgroups -> the cut): 32/8/128 fp16 B=2 ctx
    // 2048 14.98 -> 13.56, ctx 4096 17.08 -> 16.40, B=3 ctx 2048 17.12 ->
    // 14.38, ctx 4096 20.08 -> 17.82; 64/8/128 bf16 B=3 ctx 4096 21.64 ->
    // 18.62; 32/4/128 bf16 B=4 ctx 4096 17.82 -> 17.14; longer contexts and
    // larger batches unchanged, a ragged 3-sequence batch +0.3 us.
    const int64_t segments = cdiv(grid, lunits);
    if (!pair_balanced && p->heads_per_wg <= kFusedMergeMaxHeads && segments > kFusedMaxSegments &&
        lunits * kFusedMaxSegments >= cus / 2 && pages < kMinSegmentPages * segments) {
      grid = std::min(grid, lunits * std::max<int64_t>(kFusedMaxSegments, cdiv(pages, kMinSegmentPages)));
    }
    // Workspace: a partial slot per workgroup and list unit (two when paired).
    auto set_grid = [&](int64_t g) {
      p->grid = static_cast<int>(g);
      const size_t slots = (static_cast<size_t>(g) + static_cast<size_t>(lunits)) * (pair_balanced ? 2 : 1);
      p->o_bytes = align_up(slots * p->heads_per_wg * head_dim * sizeof(float));
      p->ws_bytes = p->o_bytes + align_up(slots * p->heads_per_wg * sizeof(float));
    };
    set_grid(grid);
    if (units >= cus && lunits >= cus) {
      // A full batch: one workgroup per list unit (the uniform cut on an even
      // batch) when that still gives every CU a workgroup, unless that
      // workspace would be large.
      const int64_t each = std::max<int64_t>(1, std::min<int64_t>(lunits, cdiv(upper, kMinPagesPerBalancedWg)));
      const Plan keep = *p;
      set_grid(each);
      if (p->ws_bytes > kAutoBalanceMaxWorkspace) *p = keep;
    }
    p->paired = pair_balanced;
    p->num_splits = 0;
    p->pages_per_split = 0;
    // A full batch balanced by default keeps uniform splits when the balanced
    // workspace would be large.
    const bool by_default = !requested && units >= cus && full_batch_choice < 0;
    if (!by_default || p->ws_bytes <= kAutoBalanceMaxWorkspace) return ok();
    p->grid = 0;
    p->paired = false;
  }
  int s = num_splits;
  if (s == 0) {
    // Enough splits for about one workgroup per compute unit, each split at
    // least kMinPagesPerSplit pages, never more than 64 (the rule of
    // choose_num_splits, kernel_lab/triton_kernels/paged_attention.py:169-173,
    // retuned on MI355X: one 4-wave workgroup per CU beat two for every split
    // count measured, and splits under 16 pages lose more to the merge than
    // they gain in parallelism). A single sequence takes splits of 8 pages:
    // 32/8/128 fp16 B=1 (events, us) ctx 512 S=4 9.9 vs S=2 10.9, ctx 1024
    // S=8 10.0 vs S=4 11.2, ctx 4096 S=32 13.2 vs S=16 13.4-13.5.
    const int64_t wanted = cdiv(cus, units);
    const int min_pages = batch == 1 && !partials ? kMinPagesPerSingleSplit : kMinPagesPerSplit;
    const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(cdiv(pages, min_pages), kMaxPlannedSplits));
    s = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(wanted, cap)));
  }
  // Normalise: drop splits no sequence can reach (paged_attention.py:210-211).
  const int pps = static_cast<int>(cdiv(pages, s));
  s = static_cast<int>(cdiv(pages, pps));
  p->num_splits = s;
  p->pages_per_split = pps;
  // Two adjacent KV heads per 8-wave workgroup when the pairs alone give
  // every CU a workgroup (one 8-wave workgroup per CU is the register budget)
  // and the 4-wave kernel fits two waves per SIMD (head_dim <= 128).
  p->paired = mfma && opt.pairing() && num_kv_heads % 2 == 0 && head_dim <= 128 && units * s / 2 >= cus;
  if (s > 1 || partials) {
    const size_t rows = static_cast<size_t>(batch) * num_q_heads * s;
    p->o_bytes = align_up(rows * head_dim * sizeof(float));
    p->ws_bytes = p->o_bytes + align_up(rows * sizeof(float));
  } else {
    p->o_bytes = 0;
    p->ws_bytes = 0;
  }
  return ok();
}

// The last decode plan made on this thread and the arguments it was made
// for: a caller that sizes the workspace with kl_paged_decode_plan and then
// launches with the same arguments (the PyTorch operator does) plans once.
struct PlanMemo {
  static constexpr int kKeyLen = 11;
  int key[kKeyLen] = {};
  Plan plan{};
  bool valid = false;
};
thread_local PlanMemo g_plan_memo;

int decode_plan(const Options& opt, kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                int page_size, int max_pages, int num_splits, int cu_count, bool use_mfma, Plan* p) {
  const int key[PlanMemo::kKeyLen] = {static_cast<int>(opt.bits), static_cast<int>(dtype), batch, num_q_heads,
                                      num_kv_heads, head_dim, page_size, max_pages, num_splits, cu_count,
                                      use_mfma ? 1 : 0};
  PlanMemo& m = g_plan_memo;
  if (m.valid && std::equal(key, key + PlanMemo::kKeyLen, m.key)) {
    *p = m.plan;
    return ok();
  }
  const int st = make_plan(opt, dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits,
                           cu_count, p, false, use_mfma);
  if (st != KL_OK) return st;
  std::copy(key, key + PlanMemo::kKeyLen, m.key);
  m.plan = *p;
  m.valid = true;
  return st;
}

template <int N>
using IntC = std::integral_constant<int, N>;

// Calls f(IntC<D>, IntC<NT>) for the MFMA kernel instance that serves
// head_dim and the workgroup's head tiling (NT = 2 for more than 16 query
// heads per workgroup).
template <typename F>
int dispatch_mfma(int head_dim, int heads_per_wg, F&& f) {
  const bool two = heads_per_wg > 16;
  switch (head_dim) {
    case 32:
      return two ? f(IntC<32>{}, IntC<2>{}) : f(IntC<32>{}, IntC<1>{});
    case 64:
      return two ? f(IntC<64>{}, IntC<2>{}) : f(IntC<64>{}, IntC<1>{});
    case 128:
      return two ? f(IntC<128>{}, IntC<2>{}) : f(IntC<128>{}, IntC<1>{});
    case 256:
      return f(IntC<256>{}, IntC<1>{});
  }
  return fail(KL_ERR_UNSUPPORTED, "no MFMA kernel for this head_dim");
}

// FP8 caches need 16-token blocks of at least one full 16-byte load per lane:
// head_dim >= 64.
template <typename KVF, int D>
constexpr bool mfma_instance_exists() {
  return KVF::kBytes == 2 || D >= 64;
}

template <typename E>
int launch_valu(const DecodeArgs& a, int head_dim, unsigned grid, hipStream_t stream) {
#define KL_VALU_CASE(DIM)                                                                     \
  case DIM:                                                                                   \
    if constexpr (DIM / (16 / E::kBytes) >= 1 && DIM / (16 / E::kBytes) <= 64) {              \
      switch (a.heads_per_wg) {                                                               \
        case 1:                                                                               \
          decode_valu_kernel<E, DIM, 1><<<grid, kThreads, 0, stream>>>(a);                    \
          return KL_OK;                                                                       \
        case 2:                                                                               \
          decode_valu_kernel<E, DIM, 2><<<grid, kThreads, 0, stream>>>(a);                    \
          return KL_OK;                                                                       \
        case 4:                                                                               \
          decode_valu_kernel<E, DIM, 4><<<grid, kThreads, 0, stream>>>(a);                    \
          return KL_OK;                                                                       \
        default:                                                                              \
          decode_valu_kernel<E, DIM, 8><<<grid, kThreads, 0, stream>>>(a);                    \
          return KL_OK;                                                                       \
      }                                                                                       \
    }                                                                                         \
    break;
  switch (head_dim) {
    KL_VALU_CASE(16)
    KL_VALU_CASE(32)
    KL_VALU_CASE(64)
    KL_VALU_CASE(128)
    KL_VALU_CASE(256)
  }
#undef KL_VALU_CASE
  return fail(KL_ERR_UNSUPPORTED, "no kernel for this head_dim");
}

// grid: the number of units (sequences x KV heads x head groups x splits);
// paired launches take two units per workgroup, so grid must then be even.
template <typename E, typename KVF>
int launch_uniform_mfma(const DecodeArgs& a, int head_dim, unsigned grid, hipStream_t stream) {
  if (a.paired && (grid % 2 != 0 || a.num_kv_heads % 2 != 0)) {
    return fail(KL_ERR_UNSUPPORTED, "paired decode launch needs an even number of KV heads");
  }
  return dispatch_mfma(head_dim, a.heads_per_wg, [&](auto d, auto nt) -> int {
    constexpr int D = decltype(d)::value, NT = decltype(nt)::value;
    if constexpr (mfma_instance_exists<KVF, D>()) {
      if (a.paired) {
        // head_dim 256 is never paired: its segment needs more than the
        // 256 registers per lane an 8-wave workgroup leaves.
        if constexpr (D <= 128) {
          decode_mfma_paired_kernel<E, KVF, D, NT><<<grid / 2, 2 * kThreads, 0, stream>>>(a);
        } else {
          return fail(KL_ERR_UNSUPPORTED, "paired decode needs head_dim <= 128");
        }
      } else {
        decode_mfma_kernel<E, KVF, D, NT><<<grid, kThreads, 0, stream>>>(a);
      }
      return KL_OK;
    } else {
      return fail(KL_ERR_UNSUPPORTED, "an FP8 cache needs head_dim 64, 128 or 256");
    }
  });
}

// The balanced cut's charge for starting a segment (list_prefix), in pages of
// one list unit: the bytes a workgroup streams in about the time a segment's
// start and end take (first K/V round trip after the schedule, cross-wave
// merge: kSegmentStartBytes) plus the partial it adds (its fp32 rows, written
// by the segment and read back by the merge), over one page's K and V bytes.
int balanced_charge(int page_size, int head_dim, int kv_bytes, int paired, int heads_per_wg) {
  const int halves = paired ? 2 : 1;
  const int64_t page_bytes = static_cast<int64_t>(page_size) * head_dim * kv_bytes * 2 * halves;
  const int64_t partial_bytes = static_cast<int64_t>(heads_per_wg) * head_dim * 4 * halves;
  return static_cast<int>(
      std::min<int64_t>(kMaxSegmentCharge, cdiv(kSegmentStartBytes + 2 * partial_bytes, page_bytes)));
}

template <typename E, typename KVF>
int launch_balanced(DecodeArgs a, int head_dim, hipStream_t stream) {
  const unsigned grid = static_cast<unsigned>(a.grid);
  const int64_t units = static_cast<int64_t>(a.batch) * a.num_kv_heads * a.head_groups;
  // The even-batch start needs one workgroup per list unit and the batch's
  // seq_lens in one wave-wide scan.
  const int64_t lunits = a.paired ? units / 2 : units;
  a.even_start = a.grid == lunits && a.batch <= 64 * kScanChunks ? 1 : 0;
  a.seg_charge = balanced_charge(a.page_size, head_dim, KVF::kBytes, a.paired, a.heads_per_wg);
  a.arrivals = fused_merge_counters(a, units, stream);
  int st = dispatch_mfma(head_dim, a.heads_per_wg, [&](auto d, auto nt) -> int {
    constexpr int D = decltype(d)::value, NT = decltype(nt)::value;
    if constexpr (mfma_instance_exists<KVF, D>()) {
      if (a.paired) {
        // One head tile and head_dim <= 128: beyond that the segment needs
        // more than the 256 registers per lane of an 8-wave workgroup.
        if constexpr (D <= 128 && NT == 1) {
          decode_mfma_balanced_kernel<E, KVF, D, NT, 2><<<grid, 2 * kThreads, 0, stream>>>(a);
        } else {
          return fail(KL_ERR_UNSUPPORTED, "paired balanced decode needs head_dim <= 128 and <= 16 heads per workgroup");
        }
      } else {
        decode_mfma_balanced_kernel<E, KVF, D, NT, 1><<<grid, kThreads, 0, stream>>>(a);
      }
      return KL_OK;
    } else {
      return fail(KL_ERR_UNSUPPORTED, "an FP8 cache needs head_dim 64, 128 or 256");
    }
  });
  if (st != KL_OK) return st;
  st = check_launch("paged decode balanced kernel launch");
  if (st != KL_OK) return st;
  g_last_merge = a.arrivals != nullptr ? KL_MERGE_IN_KERNEL : KL_MERGE_KERNEL;
  if (a.arrivals != nullptr) return st;
  decode_merge_balanced_kernel<E>
      <<<static_cast<unsigned>(static_cast<int64_t>(a.batch) * a.num_q_heads), 64, 0, stream>>>(a, head_dim);
  return check_launch("paged decode balanced merge kernel launch");
}

// E: query / output format; KVF: cache format (E, or Fp8E4M3 on the MFMA path).
template <typename E, typename KVF>
int launch_typed(DecodeArgs& a, int head_dim, bool mfma, hipStream_t stream) {
  if constexpr (std::is_same_v<E, F32>) {
    if (mfma || a.grid > 0) return fail(KL_ERR_UNSUPPORTED, "fp32 runs on the VALU path only");
  }
  if (a.grid > 0) {
    if constexpr (!std::is_same_v<E, F32>) return launch_balanced<E, KVF>(a, head_dim, stream);
  }
  const int64_t wgs = static_cast<int64_t>(a.batch) * a.num_kv_heads * a.head_groups * a.num_splits;
  if (wgs > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "too many workgroups");
  if (mfma && a.num_splits > 1) {
    a.arrivals = fused_merge_counters(a, static_cast<int64_t>(a.batch) * a.num_kv_heads * a.head_groups, stream);
  }
  int st;
  if constexpr (!std::is_same_v<E, F32>) {
    st = mfma ? launch_uniform_mfma<E, KVF>(a, head_dim, static_cast<unsigned>(wgs), stream)
              : launch_valu<E>(a, head_dim, static_cast<unsigned>(wgs), stream);
  } else {
    st = launch_valu<E>(a, head_dim, static_cast<unsigned>(wgs), stream);
  }
  if (st != KL_OK) return st;
  st = check_launch("paged decode split kernel launch");
  if (st != KL_OK) return st;
  g_last_merge = a.num_splits <= 1 ? KL_MERGE_NONE : a.arrivals != nullptr ? KL_MERGE_IN_KERNEL : KL_MERGE_KERNEL;
  if (a.num_splits > 1 && a.arrivals == nullptr) {
    decode_merge_kernel<E><<<static_cast<unsigned>(static_cast<int64_t>(a.batch) * a.num_q_heads), 64, 0, stream>>>(
        a, head_dim);
    st = check_launch("paged decode merge kernel launch");
  }
  return st;
}

}  // namespace
}  // namespace kl

extern "C" int kl_paged_decode_plan(kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                    int page_size, int max_pages, int num_splits, int cu_count,
                                    int* out_num_splits, size_t* out_workspace) {
  using namespace kl;
  if (cu_count <= 0) cu_count = current_cu_count();
  const Options opt = options();
  Plan p;
  const int st = decode_plan(opt, dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages,
                             num_splits, cu_count, !opt.force_valu(), &p);
  if (st != KL_OK) return st;
  if (out_num_splits) *out_num_splits = p.num_splits;
  if (out_workspace) *out_workspace = p.ws_bytes;
  return ok();
}

namespace kl {
namespace {

// Shared body of the two decode entry points. kv8: the caches hold OCP e4m3
// codes with per-KV-head fp32 scales; otherwise they hold `dtype` like q.
int decode_entry(kl_dtype dtype, bool kv8, void* out, const void* q, const void* k_cache, const void* v_cache,
                 const float* k_scale, const float* v_scale, const int32_t* block_table, const int32_t* seq_lens,
                 int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                 int64_t block_table_stride, int max_pages, float scale, int num_splits, void* workspace,
                 size_t workspace_bytes, hipStream_t stream) {
  g_last_merge = KL_MERGE_NONE;
  if (batch == 0) return ok();
  if (kv8) {
    if (dtype != KL_DTYPE_F16 && dtype != KL_DTYPE_BF16) {
      return fail(KL_ERR_UNSUPPORTED, "an FP8 cache needs fp16 or bf16 queries");
    }
    if (!mfma_path(dtype, head_dim, page_size) || head_dim < 64) {
      return fail(KL_ERR_UNSUPPORTED, "an FP8 cache needs head_dim 64, 128 or 256 and page_size a multiple of 16");
    }
    if (!k_scale || !v_scale) return fail(KL_ERR_INVALID_ARGUMENT, "k_scale and v_scale must be non-null");
  }
  const Options opt = options();
  const bool use_mfma = kv8 || !opt.force_valu();
  Plan p;
  int st = decode_plan(opt, dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages, num_splits,
                       current_cu_count(), use_mfma, &p);
  if (st != KL_OK) return st;
  if (!out || !q || !k_cache || !v_cache || !block_table || !seq_lens) {
    return fail(KL_ERR_INVALID_ARGUMENT, "out, q, k_cache, v_cache, block_table and seq_lens must be non-null");
  }
  if (max_pages < 1) return fail(KL_ERR_INVALID_ARGUMENT, "max_pages must be >= 1");
  if (block_table_stride < max_pages && batch > 1) {
    return fail(KL_ERR_INVALID_ARGUMENT, "block_table_stride must be >= max_pages");
  }
  const uintptr_t align_mask = 15;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(out)) & align_mask) {
    return fail(KL_ERR_INVALID_ARGUMENT, "q, out and the caches must be 16-byte aligned");
  }
  if (p.ws_bytes > 0 && (workspace == nullptr || workspace_bytes < p.ws_bytes)) {
    return fail(KL_ERR_WORKSPACE, "workspace smaller than kl_paged_decode_plan reported");
  }
  if ((reinterpret_cast<uintptr_t>(workspace) & align_mask) != 0) {
    return fail(KL_ERR_INVALID_ARGUMENT, "workspace must be 16-byte aligned");
  }

  DecodeArgs a;
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.out = out;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.k_scale = kv8 ? k_scale : nullptr;
  a.v_scale = kv8 ? v_scale : nullptr;
  a.o_part = static_cast<float*>(workspace);
  a.lse_part = workspace ? reinterpret_cast<float*>(static_cast<char*>(workspace) + p.o_bytes) : nullptr;
  a.bt_stride = block_table_stride;
  a.page_stride = static_cast<int64_t>(page_size) * num_kv_heads * head_dim;
  const int64_t token_stride = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (token_stride > 0x7fffffffLL / 64) return fail(KL_ERR_UNSUPPORTED, "num_kv_heads * head_dim too large");
  a.token_stride = static_cast<int>(token_stride);
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  set_page_size(a, page_size);
  a.max_pages = max_pages;
  a.num_splits = p.num_splits;
  a.pages_per_split = p.pages_per_split;
  a.head_groups = p.head_groups;
  a.grid = p.grid;
  a.even_start = 0;  // set by launch_balanced
  a.seg_charge = 0;
  a.heads_per_wg = p.heads_per_wg;
  a.scale_log2 = scale * kLog2e;
  a.q_fold = a.group;
  a.q_heads = num_q_heads;
  a.force_partial = 0;
  a.paired = p.paired ? 1 : 0;
  a.arrivals = nullptr;

  const bool mfma = use_mfma && mfma_path(dtype, head_dim, page_size);
  switch (dtype) {
    case KL_DTYPE_F32:
      return launch_typed<F32, F32>(a, head_dim, false, stream);
    case KL_DTYPE_F16:
      return kv8 ? launch_typed<F16, Fp8E4M3>(a, head_dim, true, stream)
                 : launch_typed<F16, F16>(a, head_dim, mfma, stream);
    case KL_DTYPE_BF16:
      return kv8 ? launch_typed<BF16, Fp8E4M3>(a, head_dim, true, stream)
                 : launch_typed<BF16, BF16>(a, head_dim, mfma, stream);
  }
  return fail(KL_ERR_UNSUPPORTED, "dtype must be f32, f16 or bf16");
}

}  // namespace
}  // namespace kl

extern "C" int kl_paged_decode_attention(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                         const void* v_cache, const int32_t* block_table, const int32_t* seq_lens,
                                         int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                         int64_t block_table_stride, int max_pages, float scale, int num_splits,
                                         void* workspace, size_t workspace_bytes, kl_stream_t stream) {
  return kl::decode_entry(dtype, false, out, q, k_cache, v_cache, nullptr, nullptr, block_table, seq_lens, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, block_table_stride, max_pages, scale,
                          num_splits, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int kl_paged_decode_last_merge(void) { return kl::g_last_merge; }

extern "C" int kl_paged_decode_reload_options(void) {
  kl::g_option_bits.store(kl::read_option_bits(), std::memory_order_relaxed);
  return kl::ok();
}

// --------------------------------------------- no-allocation decode entry point
//
// The split workspace of kl_paged_decode_attention (fp32 partial outputs and
// their log2-sum-exps) for callers that cannot allocate device memory, in a
// library-owned array. 16 MiB holds every split the planner chooses by itself
// (num_splits 0): the planner keeps a full batch's balanced workspace within
// kAutoBalanceMaxWorkspace (this size) and falls back to uniform splits
// beyond it; smaller batches need at most about 8.5 MB (511 balanced slots of
// 32 heads x 129 floats or 16 heads x 257). Each device holds its own copy until the process
// ends. No byte of it has to start at zero: a merge reads only partials that
// the same call wrote before. Calls that overlap on one device share it, so
// they race.
constexpr size_t kScratchBytes = size_t{16} << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace kl {
namespace {

constexpr int kMaxScratchDevices = 64;

// Device address of the current device's `scratch`. Host code never uses the
// array's own name as an address (it is a host-side stand-in): the runtime
// reports each device's copy once, with that device current, and the address
// is kept per device. Null (with the error recorded) if the lookup fails.
void* scratch_for_current_device() {
  static std::mutex mu;
  static void* addr[kMaxScratchDevices] = {};
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    fail_hip(e, "hipGetDevice");
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxScratchDevices) {
    fail(KL_ERR_UNSUPPORTED, "device index beyond the no-allocation entry point's table");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = device_symbol_address(&p, scratch);
    if (err != hipSuccess) {
      fail_hip(err, "hipGetSymbolAddress(scratch)");
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

}  // namespace
}  // namespace kl

extern "C" int kl_paged_decode_attention_noalloc(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                                 const void* v_cache, const int32_t* block_table,
                                                 const int32_t* seq_lens, int batch, int num_q_heads,
                                                 int num_kv_heads, int head_dim, int page_size,
                                                 int64_t block_table_stride, int max_pages, float scale,
                                                 int num_splits, kl_stream_t stream) {
  using namespace kl;
  // Every return below, including a refusal, reports no merge.
  g_last_merge = KL_MERGE_NONE;
  // Set-up first: the device's scratch address is looked up on the first call
  // on each device, whatever this call needs.
  void* ws = scratch_for_current_device();
  if (ws == nullptr) return KL_ERR_HIP;
  if (batch == 0) return ok();
  int splits = 0;
  size_t need = 0;
  const int st = kl_paged_decode_plan(dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, max_pages,
                                      num_splits, 0, &splits, &need);
  if (st != KL_OK) return st;
  if (need > kScratchBytes) {
    char msg[200];
    std::snprintf(msg, sizeof(msg),
                  "this split plan needs %zu bytes of workspace; the no-allocation entry point holds %zu "
                  "(use kl_paged_decode_attention with a caller workspace, or fewer splits)",
                  need, kScratchBytes);
    return fail(KL_ERR_WORKSPACE, msg);
  }
  return kl::decode_entry(dtype, false, out, q, k_cache, v_cache, nullptr, nullptr, block_table, seq_lens, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, block_table_stride, max_pages, scale,
                          num_splits, need > 0 ? ws : nullptr, need > 0 ? kScratchBytes : 0,
                          reinterpret_cast<hipStream_t>(stream));
}

extern "C" int kl_paged_decode_attention_fp8(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                             const void* v_cache, const float* k_scale, const float* v_scale,
                                             const int32_t* block_table, const int32_t* seq_lens, int batch,
                                             int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                             int64_t block_table_stride, int max_pages, float scale,
                                             int num_splits, void* workspace, size_t workspace_bytes,
                                             kl_stream_t stream) {
  return kl::decode_entry(dtype, true, out, q, k_cache, v_cache, k_scale, v_scale, block_table, seq_lens, batch,
                          num_q_heads, num_kv_heads, head_dim, page_size, block_table_stride, max_pages, scale,
                          num_splits, workspace, workspace_bytes, reinterpret_cast<hipStream_t>(stream));
}

// ------------------------------------------------------- cascade entry points

namespace kl {
namespace {

struct CascadePlan {
  Plan pre;        // shared-prefix pass (batch 1, folded group)
  Plan suf;        // per-sequence pass
  size_t pre_bytes;
  size_t ws_bytes;
};

int cascade_plan(kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                 int prefix_pages, int max_pages, int cu_count, CascadePlan* cp) {
  if (dtype != KL_DTYPE_F16 && dtype != KL_DTYPE_BF16) {
    return fail(KL_ERR_UNSUPPORTED, "cascade decode needs fp16 or bf16");
  }
  if (!mfma_path(dtype, head_dim, page_size)) {
    return fail(KL_ERR_UNSUPPORTED, "cascade decode needs head_dim 32, 64, 128 or 256 and page_size a multiple of 16");
  }
  if (batch < 0 || num_kv_heads <= 0 || num_q_heads <= 0 || prefix_pages < 0 || max_pages < 0) {
    return fail(KL_ERR_INVALID_ARGUMENT, "batch, heads and page counts must be non-negative");
  }
  if (num_q_heads % num_kv_heads != 0) {
    return fail(KL_ERR_INVALID_ARGUMENT, "num_q_heads must be a multiple of num_kv_heads");
  }
  const int64_t folded = static_cast<int64_t>(std::max(batch, 1)) * (num_q_heads / num_kv_heads);
  if (folded * num_kv_heads > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "batch * num_q_heads too large");
  const Options opt = options();
  int st = make_plan(opt, dtype, 1, static_cast<int>(folded * num_kv_heads), num_kv_heads, head_dim, page_size,
                     std::max(prefix_pages, 1), 0, cu_count, &cp->pre, true);
  if (st != KL_OK) return st;
  st = make_plan(opt, dtype, std::max(batch, 1), num_q_heads, num_kv_heads, head_dim, page_size,
                 std::max(max_pages, 1), 0, cu_count, &cp->suf, true);
  if (st != KL_OK) return st;
  cp->pre_bytes = align_up(cp->pre.ws_bytes);
  cp->ws_bytes = cp->pre_bytes + cp->suf.ws_bytes;
  return ok();
}

template <typename E>
int cascade_launch(const DecodeArgs& base, const CascadePlan& cp, const int32_t* prefix_block_table,
                   const int32_t* prefix_len, int prefix_pages, const int32_t* block_table, const int32_t* seq_lens,
                   int64_t bt_stride, int max_pages, char* ws, int head_dim, hipStream_t stream) {
  const int batch = base.batch;
  const int num_q_heads = base.num_q_heads;
  const int group = base.group;
  if (prefix_pages > 0) {
    DecodeArgs a = base;
    a.block_table = prefix_block_table;
    a.seq_lens = prefix_len;
    a.bt_stride = prefix_pages;
    a.batch = 1;
    a.group = batch * group;
    a.num_q_heads = a.num_kv_heads * a.group;
    a.max_pages = prefix_pages;
    a.num_splits = cp.pre.num_splits;
    a.pages_per_split = cp.pre.pages_per_split;
    a.head_groups = cp.pre.head_groups;
    a.heads_per_wg = cp.pre.heads_per_wg;
    a.o_part = reinterpret_cast<float*>(ws);
    a.lse_part = reinterpret_cast<float*>(ws + cp.pre.o_bytes);
    a.paired = cp.pre.paired ? 1 : 0;
    const int64_t wgs = static_cast<int64_t>(a.num_kv_heads) * a.head_groups * a.num_splits;
    if (wgs > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "too many workgroups");
    int st = launch_uniform_mfma<E, E>(a, head_dim, static_cast<unsigned>(wgs), stream);
    if (st != KL_OK) return st;
    st = check_launch("cascade prefix pass launch");
    if (st != KL_OK) return st;
  }
  DecodeArgs a = base;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.bt_stride = bt_stride;
  a.max_pages = max_pages;
  a.num_splits = cp.suf.num_splits;
  a.pages_per_split = cp.suf.pages_per_split;
  a.head_groups = cp.suf.head_groups;
  a.heads_per_wg = cp.suf.heads_per_wg;
  a.o_part = reinterpret_cast<float*>(ws + cp.pre_bytes);
  a.lse_part = reinterpret_cast<float*>(ws + cp.pre_bytes + cp.suf.o_bytes);
  a.paired = cp.suf.paired ? 1 : 0;
  const int64_t wgs = static_cast<int64_t>(batch) * a.num_kv_heads * a.head_groups * a.num_splits;
  if (wgs > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "too many workgroups");
  int st = launch_uniform_mfma<E, E>(a, head_dim, static_cast<unsigned>(wgs), stream);
  if (st != KL_OK) return st;
  st = check_launch("cascade suffix pass launch");
  if (st != KL_OK) return st;

  CascadeArgs c;
  c.p_o = reinterpret_cast<const float*>(ws);
  c.p_lse = reinterpret_cast<const float*>(ws + cp.pre.o_bytes);
  c.prefix_len = prefix_len;
  c.prefix_pages = prefix_pages;
  c.p_splits = cp.pre.num_splits;
  c.p_pps = cp.pre.pages_per_split;
  c.s_o = a.o_part;
  c.s_lse = a.lse_part;
  c.seq_lens = seq_lens;
  c.max_pages = max_pages;
  c.s_splits = cp.suf.num_splits;
  c.s_pps = cp.suf.pages_per_split;
  c.out = base.out;
  c.batch = batch;
  c.num_q_heads = num_q_heads;
  c.group = group;
  c.page_size = base.page_size;
  cascade_merge_kernel<E><<<static_cast<unsigned>(static_cast<int64_t>(batch) * num_q_heads), 64, 0, stream>>>(
      c, head_dim);
  return check_launch("cascade merge kernel launch");
}

}  // namespace
}  // namespace kl

extern "C" int kl_cascade_decode_plan(kl_dtype dtype, int batch, int num_q_heads, int num_kv_heads, int head_dim,
                                      int page_size, int prefix_pages, int max_pages, int cu_count,
                                      size_t* out_workspace) {
  using namespace kl;
  if (cu_count <= 0) cu_count = current_cu_count();
  CascadePlan cp;
  const int st = cascade_plan(dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, prefix_pages, max_pages,
                              cu_count, &cp);
  if (st != KL_OK) return st;
  if (out_workspace) *out_workspace = cp.ws_bytes;
  return ok();
}

extern "C" int kl_cascade_decode_attention(kl_dtype dtype, void* out, const void* q, const void* k_cache,
                                           const void* v_cache, const int32_t* prefix_block_table,
                                           const int32_t* prefix_len, int prefix_pages,
                                           const int32_t* block_table, const int32_t* seq_lens, int batch,
                                           int num_q_heads, int num_kv_heads, int head_dim, int page_size,
                                           int64_t block_table_stride, int max_pages, float scale, void* workspace,
                                           size_t workspace_bytes, kl_stream_t stream) {
  using namespace kl;
  if (batch == 0) return ok();
  CascadePlan cp;
  int st = cascade_plan(dtype, batch, num_q_heads, num_kv_heads, head_dim, page_size, prefix_pages, max_pages,
                        current_cu_count(), &cp);
  if (st != KL_OK) return st;
  if (!out || !q || !k_cache || !v_cache || !block_table || !seq_lens || !prefix_len ||
      (prefix_pages > 0 && !prefix_block_table)) {
    return fail(KL_ERR_INVALID_ARGUMENT, "tensor pointers must be non-null");
  }
  if (max_pages < 1) return fail(KL_ERR_INVALID_ARGUMENT, "max_pages must be >= 1");
  if (block_table_stride < max_pages && batch > 1) {
    return fail(KL_ERR_INVALID_ARGUMENT, "block_table_stride must be >= max_pages");
  }
  const uintptr_t align_mask = 15;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(workspace)) & align_mask) {
    return fail(KL_ERR_INVALID_ARGUMENT, "q, out, the caches and the workspace must be 16-byte aligned");
  }
  if (workspace == nullptr || workspace_bytes < cp.ws_bytes) {
    return fail(KL_ERR_WORKSPACE, "workspace smaller than kl_cascade_decode_plan reported");
  }
  const int64_t token_stride = static_cast<int64_t>(num_kv_heads) * head_dim;
  if (token_stride > 0x7fffffffLL / 64) return fail(KL_ERR_UNSUPPORTED, "num_kv_heads * head_dim too large");

  DecodeArgs a{};
  a.q = q;
  a.k = k_cache;
  a.v = v_cache;
  a.out = out;
  a.k_scale = nullptr;
  a.v_scale = nullptr;
  a.page_stride = static_cast<int64_t>(page_size) * num_kv_heads * head_dim;
  a.token_stride = static_cast<int>(token_stride);
  a.batch = batch;
  a.num_q_heads = num_q_heads;
  a.num_kv_heads = num_kv_heads;
  a.group = num_q_heads / num_kv_heads;
  set_page_size(a, page_size);
  a.grid = 0;
  a.paired = 0;
  a.arrivals = nullptr;
  a.scale_log2 = scale * kLog2e;
  a.q_fold = a.group;
  a.q_heads = num_q_heads;
  a.force_partial = 1;
  const auto s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  return dtype == KL_DTYPE_F16
             ? cascade_launch<F16>(a, cp, prefix_block_table, prefix_len, prefix_pages, block_table, seq_lens,
                                   block_table_stride, max_pages, ws, head_dim, s)
             : cascade_launch<BF16>(a, cp, prefix_block_table, prefix_len, prefix_pages, block_table, seq_lens,
                                    block_table_stride, max_pages, ws, head_dim, s);
}
