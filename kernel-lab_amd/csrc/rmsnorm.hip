// RMSNorm and fused residual-add + RMSNorm for gfx950.
//
// Math (reference: csrc/rmsnorm.cu:17-62 and kernel_lab/reference.py:13-30):
//   res = dtype(f32(x) + f32(res))                  (fused variant only)
//   rstd = 1 / sqrt(sum(f32(res)^2) / hidden + eps)
//   out = dtype((f32(res) * rstd) * f32(weight))
// The sum is rounded to the storage dtype before it is normalised, because
// that rounded value is what the residual stream keeps; the residual output is
// therefore bit-identical to PyTorch's.
//
// Design: one workgroup per row. Each thread loads its share of the row as
// 16-byte packs, strided by the workgroup size so every wave load is one
// contiguous 1 KiB span, and keeps the values in registers. The sum of squares
// is reduced within each wave by DPP, across waves through LDS with one
// barrier, and the output is written from registers: one read of x and the
// residual, one write of the residual and the output, nothing re-read.
// Rows too wide for the register budget use a two-pass variant that keeps the
// rounded sum in LDS (and forms it again for what LDS cannot hold).
#include <algorithm>

#include "hip_common.h"
#include "kl_internal.h"

namespace kl {
namespace {

template <typename S, int N>
struct alignas(sizeof(S) * N) Pack {
  S v[N];
};

// Pack loads and stores keep the default cache policy: measured on MI355X for
// this read/write mix, non-temporal stores lose ~10% of HBM bandwidth and
// non-temporal loads ~7%.
template <typename S, int N>
__device__ __forceinline__ Pack<S, N> load_pack(const Pack<S, N>* p) {
  return *p;
}

// Packs per thread the launch aims for (threads = packs / 2, in whole waves,
// 64..1024): measured on MI355X at hidden 8192 bf16, one, four and eight
// 16-byte packs per tensor per thread were slower than two.
constexpr int kPacksPerThread = 2;

template <typename S, int N>
__device__ __forceinline__ void store_pack(Pack<S, N>* p, const Pack<S, N>& v) {
  *p = v;
}

constexpr int kMaxThreads = 1024;

// Workgroup-wide sum; every thread receives the same value. `scratch` holds one
// float per wave. Wave sums are added in wave order, so the result is
// deterministic.
__device__ __forceinline__ float block_sum(float v, float* scratch) {
  const float w = wave_sum(v);
  const int nw = blockDim.x >> 6;
  if (__lane_id() == 0) scratch[threadIdx.x >> 6] = w;
  __syncthreads();
  float total = 0.0f;
  for (int i = 0; i < nw; ++i) total += scratch[i];
  return total;
}

__device__ __forceinline__ float inv_rms(float sum_sq, int hidden, float eps) {
  // Division and square root are IEEE-rounded here (no fast-math), matching
  // torch.rsqrt on the CPU, which computes 1 / sqrt(x).
  return 1.0f / sqrtf(sum_sq / static_cast<float>(hidden) + eps);
}

// Register-resident single pass. Thread t owns packs t, t + NT, ..., so NPACK
// loads per tensor per thread; NT * NPACK * VEC >= hidden. Every load is
// issued unconditionally (indexes past the row are clamped to its last pack
// and their values masked to zero), so all of a thread's loads are in flight
// together; a branch per pack would make the compiler wait for each load
// before issuing the next. Only stores are guarded.
template <typename E, int VEC, int NPACK, bool HAS_RES>
__global__ void __launch_bounds__(kMaxThreads)
    rms_norm_reg_kernel(typename E::S* __restrict__ out, const typename E::S* __restrict__ x,
                        typename E::S* __restrict__ res, const typename E::S* __restrict__ weight,
                        int hidden, int64_t x_row_stride, float eps) {
  using S = typename E::S;
  using P = Pack<S, VEC>;
  __shared__ float scratch[kMaxThreads / 64];

  const int64_t row = blockIdx.x;
  const int packs = hidden / VEC;
  const int nt = blockDim.x;
  const P* xr = reinterpret_cast<const P*>(x + row * x_row_stride);
  P* rr = HAS_RES ? reinterpret_cast<P*>(res + row * static_cast<int64_t>(hidden)) : nullptr;
  P* orow = reinterpret_cast<P*>(out + row * static_cast<int64_t>(hidden));
  const P* wr = reinterpret_cast<const P*>(weight);

  int idx[NPACK];
  bool valid[NPACK];
#pragma unroll
  for (int k = 0; k < NPACK; ++k) {
    const int p = threadIdx.x + k * nt;
    valid[k] = p < packs;
    idx[k] = valid[k] ? p : packs - 1;
  }

  P a[NPACK];
  P b[NPACK];
#pragma unroll
  for (int k = 0; k < NPACK; ++k) {
    a[k] = load_pack(xr + idx[k]);
    if constexpr (HAS_RES) b[k] = load_pack(rr + idx[k]);
  }
  // Weights are loaded before the reduction so their latency overlaps it,
  // except at NPACK = 8, where their registers beside x's and the residual's
  // would exceed the 128 a lane has at 1024 threads and spill.
  constexpr bool kEarlyWeights = NPACK <= 4;
  P w[NPACK];
  if constexpr (kEarlyWeights) {
#pragma unroll
    for (int k = 0; k < NPACK; ++k) w[k] = wr[idx[k]];
  }

  // The rounded sum stays packed across the block reduction and is widened
  // again for the output: keeping an fp32 copy live as well would need
  // NPACK * VEC more registers and spill at NPACK = 8.
  P s[NPACK];
  float sum_sq = 0.0f;
#pragma unroll
  for (int k = 0; k < NPACK; ++k) {
    if constexpr (HAS_RES) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) s[k].v[j] = E::from_f32(E::to_f32(a[k].v[j]) + E::to_f32(b[k].v[j]));
    } else {
      s[k] = a[k];
    }
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float f = E::to_f32(s[k].v[j]);
      part += f * f;
    }
    sum_sq += valid[k] ? part : 0.0f;
  }
  if constexpr (HAS_RES) {
#pragma unroll
    for (int k = 0; k < NPACK; ++k) {
      if (valid[k]) store_pack(rr + idx[k], s[k]);
    }
  }

  if constexpr (!kEarlyWeights) {
#pragma unroll
    for (int k = 0; k < NPACK; ++k) w[k] = wr[idx[k]];
  }
  const float rstd = inv_rms(block_sum(sum_sq, scratch), hidden, eps);
  if constexpr (!kEarlyWeights && sizeof(P) == 16) {
    // Keep the sums packed until here: widened ahead of the reduction (the
    // compiler's choice otherwise) they would take twice the registers.
#pragma unroll
    for (int k = 0; k < NPACK; ++k) {
      u32x4 r = __builtin_bit_cast(u32x4, s[k]);
      asm volatile("" : "+v"(r));
      s[k] = __builtin_bit_cast(P, r);
    }
  }

#pragma unroll
  for (int k = 0; k < NPACK; ++k) {
    P o;
#pragma unroll
    for (int j = 0; j < VEC; ++j) o.v[j] = E::from_f32((E::to_f32(s[k].v[j]) * rstd) * E::to_f32(w[k].v[j]));
    if (valid[k]) store_pack(orow + idx[k], o);
  }
}

// Rows wider than the register-resident kernel holds (more than 8 packs per
// thread at 1024 threads: 65,536 16-bit or 32,768 fp32 elements aligned, 8,192
// unaligned). Two passes over the row with the rounded sum kept in LDS:
//   pass 1  reads x (and the residual), forms the rounded sum, accumulates its
//           squares, and keeps the sum of the row's first kStagedPacks packs in
//           LDS (writing their residual now);
//   pass 2  normalises from LDS; packs beyond the LDS window are formed again
//           from x and the residual, whose original value is still in memory
//           because pass 1 did not write those packs, and their residual is
//           written then.
// A thread takes the same packs in both passes, so neither pass waits for
// another thread beyond the reduction's barrier; the squares are summed in the
// same order either way, so the bits do not depend on the LDS window.
constexpr int kStageBytes = 48 * 1024;

template <typename E, int VEC, bool HAS_RES>
__global__ void __launch_bounds__(kMaxThreads)
    rms_norm_staged_kernel(typename E::S* __restrict__ out, const typename E::S* __restrict__ x,
                           typename E::S* __restrict__ res, const typename E::S* __restrict__ weight,
                           int hidden, int64_t x_row_stride, float eps) {
  using S = typename E::S;
  using P = Pack<S, VEC>;
  constexpr int kStagedPacks = kStageBytes / static_cast<int>(sizeof(P));
  __shared__ P staged[kStagedPacks];
  __shared__ float scratch[kMaxThreads / 64];

  const int64_t row = blockIdx.x;
  const int packs = hidden / VEC;
  const int window = min(packs, kStagedPacks);
  const P* xr = reinterpret_cast<const P*>(x + row * x_row_stride);
  P* rr = HAS_RES ? reinterpret_cast<P*>(res + row * static_cast<int64_t>(hidden)) : nullptr;
  P* orow = reinterpret_cast<P*>(out + row * static_cast<int64_t>(hidden));
  const P* wr = reinterpret_cast<const P*>(weight);

  // The value the residual stream carries for pack p: dtype(x + residual), or x.
  auto rounded_sum = [&](int p) {
    P v = xr[p];
    if constexpr (HAS_RES) {
      const P r = rr[p];
#pragma unroll
      for (int j = 0; j < VEC; ++j) v.v[j] = E::from_f32(E::to_f32(v.v[j]) + E::to_f32(r.v[j]));
    }
    return v;
  };

  float sum_sq = 0.0f;
  for (int p = threadIdx.x; p < packs; p += blockDim.x) {
    const P v = rounded_sum(p);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float f = E::to_f32(v.v[j]);
      sum_sq += f * f;
    }
    if (p < window) {
      staged[p] = v;
      if constexpr (HAS_RES) rr[p] = v;
    }
  }
  const float rstd = inv_rms(block_sum(sum_sq, scratch), hidden, eps);

  for (int p = threadIdx.x; p < packs; p += blockDim.x) {
    P v;
    if (p < window) {
      v = staged[p];
    } else {
      v = rounded_sum(p);
      if constexpr (HAS_RES) rr[p] = v;
    }
    const P g = wr[p];
    P o;
#pragma unroll
    for (int j = 0; j < VEC; ++j) o.v[j] = E::from_f32((E::to_f32(v.v[j]) * rstd) * E::to_f32(g.v[j]));
    orow[p] = o;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename E, int VEC, bool HAS_RES>
int launch_vec(void* out, const void* x, void* res, const void* w, int64_t rows, int hidden,
               int64_t x_row_stride, float eps, hipStream_t stream) {
  using S = typename E::S;
  auto* o = static_cast<S*>(out);
  auto* xi = static_cast<const S*>(x);
  auto* r = static_cast<S*>(res);
  auto* wi = static_cast<const S*>(w);
  const int packs = hidden / VEC;
  // About kPacksPerThread packs per thread, in whole waves, 64..1024 threads.
  int threads = static_cast<int>(std::min<int64_t>(
      kMaxThreads, std::max<int64_t>(64, cdiv(cdiv(packs, kPacksPerThread), 64) * 64)));
  const int npack = static_cast<int>(cdiv(packs, threads));
  const dim3 grid(static_cast<unsigned>(rows));
  if (npack <= 1) {
    rms_norm_reg_kernel<E, VEC, 1, HAS_RES><<<grid, threads, 0, stream>>>(o, xi, r, wi, hidden, x_row_stride, eps);
  } else if (npack <= 2) {
    rms_norm_reg_kernel<E, VEC, 2, HAS_RES><<<grid, threads, 0, stream>>>(o, xi, r, wi, hidden, x_row_stride, eps);
  } else if (npack <= 4) {
    rms_norm_reg_kernel<E, VEC, 4, HAS_RES><<<grid, threads, 0, stream>>>(o, xi, r, wi, hidden, x_row_stride, eps);
  } else if (npack <= 8) {
    rms_norm_reg_kernel<E, VEC, 8, HAS_RES><<<grid, threads, 0, stream>>>(o, xi, r, wi, hidden, x_row_stride, eps);
  } else {
    rms_norm_staged_kernel<E, VEC, HAS_RES><<<grid, kMaxThreads, 0, stream>>>(o, xi, r, wi, hidden, x_row_stride, eps);
  }
  return check_launch("rms_norm kernel launch");
}

template <typename E>
int launch_typed(void* out, const void* x, void* res, const void* w, int64_t rows, int hidden,
                 int64_t x_row_stride, float eps, hipStream_t stream) {
  constexpr int kVec = 16 / E::kBytes;
  const bool vec = hidden % kVec == 0 && x_row_stride % kVec == 0 && aligned16(out) && aligned16(x) &&
                   aligned16(w) && (res == nullptr || aligned16(res));
  if (vec) {
    return res ? launch_vec<E, kVec, true>(out, x, res, w, rows, hidden, x_row_stride, eps, stream)
               : launch_vec<E, kVec, false>(out, x, res, w, rows, hidden, x_row_stride, eps, stream);
  }
  return res ? launch_vec<E, 1, true>(out, x, res, w, rows, hidden, x_row_stride, eps, stream)
             : launch_vec<E, 1, false>(out, x, res, w, rows, hidden, x_row_stride, eps, stream);
}

}  // namespace
}  // namespace kl

extern "C" int kl_rms_norm(kl_dtype dtype, void* out, const void* x, void* residual, const void* weight,
                           int64_t rows, int64_t hidden, int64_t x_row_stride, float eps,
                           kl_stream_t stream) {
  using namespace kl;
  if (rows < 0 || hidden < 0) return fail(KL_ERR_INVALID_ARGUMENT, "rows and hidden must be >= 0");
  if (rows == 0 || hidden == 0) return ok();
  if (rows > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "rows must be < 2^31");
  if (hidden > 0x7fffffffLL) return fail(KL_ERR_UNSUPPORTED, "hidden must be < 2^31");
  if (out == nullptr || x == nullptr || weight == nullptr) {
    return fail(KL_ERR_INVALID_ARGUMENT, "out, x and weight must be non-null");
  }
  if (x_row_stride < hidden && rows > 1) {
    return fail(KL_ERR_INVALID_ARGUMENT, "x_row_stride must be >= hidden");
  }
  const auto s = reinterpret_cast<hipStream_t>(stream);
  const int h = static_cast<int>(hidden);
  switch (dtype) {
    case KL_DTYPE_F32:
      return launch_typed<F32>(out, x, residual, weight, rows, h, x_row_stride, eps, s);
    case KL_DTYPE_F16:
      return launch_typed<F16>(out, x, residual, weight, rows, h, x_row_stride, eps, s);
    case KL_DTYPE_BF16:
      return launch_typed<BF16>(out, x, residual, weight, rows, h, x_row_stride, eps, s);
  }
  return fail(KL_ERR_UNSUPPORTED, "dtype must be f32, f16 or bf16");
}
