// RMSNorm and Add+RMSNorm over bf16 rows, for gfx950.
//
// Replace nanovllm/kernels/rms_norm.py (Triton, :34-111). Numerics of the torch code they stand for
// (layers/layernorm.py:20-44), bit for bit as torch computes it eagerly on the GPU:
//   rms_norm:      y = bf16(bf16(x * rstd) * w),             rstd = rsqrt(sum(x^2) * factor + eps)
//   add_rms_norm:  s = fp32(x) + fp32(r); res = bf16(s);    y = bf16(bf16(s * rstd) * w), rstd from the fp32 s
// with the sum of squares in ATen's GPU reduction order for the call's row count, factor = float(rows) /
// float(rows * n) and torch's rsqrt (common.h: torch_rsqrt, aten_norm_bw).
//
// Fast path (16-byte aligned rows; n = 64, 128 or a multiple of 256 up to 4096): LANES consecutive lanes of a
// wave64 own a row, lane j holding K 16-byte chunks at elements 8 j + 8 LANES k (a wave's loads are contiguous),
// and the row stays in registers between the reduction and the output. The chunks are exactly the data of ATen's
// threads 2 j and 2 j + 1 (+ 64 c for bw = 64 M > 64), so the sum is local work plus a LANES-wide butterfly
// (common.h t32_partial). Other widths and unaligned rows: one block of bw threads per row running ATen's
// algorithm itself (norm_kernel_generic); rows that ATen splits over the waves of a block (n >= 8192 with 8 rows
// or more) keep that kernel's two-level order, within fp32 rounding of torch's.
#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;

struct NormArgs {
  uint16_t* y;
  uint16_t* res_out;  // add_rms_norm only
  const uint16_t* x;
  const uint16_t* r;  // add_rms_norm only
  const uint16_t* w;
  int64_t rows, rows_per_group, group_stride, row_stride;  // x layout (rms_norm)
  int64_t x_stride, r_stride;                              // row strides (add_rms_norm)
  int64_t n;
  float factor, eps;  // the mean's factor (aten_mean_factor) and epsilon
  int m;              // ATen threads per row / 64 (fast path with 32 lanes); ATen threads per row (generic kernel)
  // add_rms_norm with x given as splits (1..4) fp32 partial products [splits, rows, n] (split s at xp + s * xp_split):
  // x = bf16(sum of the partials in split order), the rounding of the GEMM output they add up to
  const float* xp;
  int splits;
  int64_t xp_split;
};

// The row's sum of squares in torch's order from the lane's K chunks (layouts above), the same in every lane.
template <int LANES, int K>
__device__ __forceinline__ float row_sumsq(const float (*v)[8], int m) {
  if constexpr (LANES == 8) {  // n = 64: one element per ATen thread
    return group_sum<8>(half_sumsq8<64>(v[0]));
  } else if constexpr (LANES == 16) {  // n = 128: one vector per ATen thread, bw = 32
    return group_sum<16>(t32_partial<1, 1>(v));
  } else {
    return group_sum<32>(t32_partial_m<K>(v, m));
  }
}

template <int LANES, int K, bool ADD, bool PART = false>
__global__ __launch_bounds__(kBlock) void norm_kernel(const NormArgs a) {
  constexpr int N = LANES * K * 8, STRIDE = LANES * 8;
  const int sub = threadIdx.x % LANES;
  const int64_t row = int64_t(blockIdx.x) * (blockDim.x / LANES) + threadIdx.x / LANES;
  if (row >= a.rows) return;

  const uint16_t* xr;
  const uint16_t* rr = nullptr;
  if constexpr (ADD) {
    xr = a.x + row * a.x_stride;
    rr = a.r + row * a.r_stride;
  } else {
    const int64_t grp = row / a.rows_per_group;
    xr = a.x + grp * a.group_stride + (row - grp * a.rows_per_group) * a.row_stride;
  }

  float v[K][8];
  u32x4 raw[K], wraw[K];
  if constexpr (PART) {  // every split's chunks loaded at once, then summed in split order and rounded to bf16
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const float* xp = a.xp + row * a.n;
    f32x4 p[4][K][2];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (s < a.splits)
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            p[s][k][h] = *reinterpret_cast<const f32x4*>(xp + s * a.xp_split + k * STRIDE + sub * 8 + 4 * h);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = p[0][k][i / 4][i % 4];
#pragma unroll
      for (int s = 1; s < 4; ++s)
        if (s < a.splits)
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] += p[s][k][i / 4][i % 4];
      raw[k] = pack8(x);
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) raw[k] = load8<true>(xr + k * STRIDE + sub * 8);
  }
  // the weight is loaded up front: after the residual store the compiler could not move it past a possible alias
#pragma unroll
  for (int k = 0; k < K; ++k) wraw[k] = load8<true>(a.w + k * STRIDE + sub * 8);
  if constexpr (ADD) {
    u32x4 rraw[K];
#pragma unroll
    for (int k = 0; k < K; ++k) rraw[k] = load8<true>(rr + k * STRIDE + sub * 8);
#pragma unroll
    for (int k = 0; k < K; ++k) {
      float xf[8], rf[8];
      unpack8(raw[k], xf);
      unpack8(rraw[k], rf);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[k][i] = xf[i] + rf[i];
      store8<true>(a.res_out + row * N + k * STRIDE + sub * 8, pack8(v[k]));
    }
  } else {
#pragma unroll
    for (int k = 0; k < K; ++k) unpack8(raw[k], v[k]);
  }

  const float rstd = torch_rsqrt(row_sumsq<LANES, K>(v, a.m) * a.factor + a.eps);

#pragma unroll
  for (int k = 0; k < K; ++k) {
    float wf[8], o[8];
    unpack8(wraw[k], wf);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = round_bf16(v[k][i] * rstd) * wf[i];
    uint16_t* dst = a.y + row * N + k * STRIDE + sub * 8;
    // plain RMSNorm streams its output (measured faster); Add+RMSNorm keeps plain stores (measured slower with the
    // hint on either output)
    if constexpr (ADD) store8<true>(dst, pack8(o));
    else __builtin_nontemporal_store(pack8(o), reinterpret_cast<u32x4*>(dst));
  }
}

// Any n and alignment: one block of bw = a.m threads per row (ATen's block width for this call, <= 512) running
// ATen's reduction itself -- thread L sums its 4-element vectors L, L + bw, ... (n >= 128, n % 4 == 0) or its
// elements L, L + bw, ... in ATen's unrolled order of four accumulators (n < 128), then the block halves the
// partials down to one wave and the wave finishes with the butterfly; the output pass reads the row again (mostly
// from the cache). With bw = 0 (a row ATen splits over waves, or n >= 128 not a multiple of 4) the block is 256
// threads and the partials are plain strided sums.
template <bool ADD>
__global__ __launch_bounds__(512) void norm_kernel_generic(const NormArgs a) {
  const int64_t row = blockIdx.x;
  const uint16_t* xr;
  const uint16_t* rr = nullptr;
  if constexpr (ADD) {
    xr = a.x + row * a.x_stride;
    rr = a.r + row * a.r_stride;
  } else {
    const int64_t grp = row / a.rows_per_group;
    xr = a.x + grp * a.group_stride + (row - grp * a.rows_per_group) * a.row_stride;
  }
  auto val = [&](int64_t i) {
    float s = bf16_to_f32(xr[i]);
    if constexpr (ADD) s += bf16_to_f32(rr[i]);
    return s;
  };
  const int bw = blockDim.x, L = threadIdx.x;
  const bool exact = a.m > 0;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (exact && a.n >= 128) {
    for (int64_t vi = L; vi < a.n / 4; vi += bw)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = val(4 * vi + i);
        acc[i] += s * s;
      }
  } else if (exact) {
    int64_t idx = L;
    for (; idx + 3 * bw < a.n; idx += 4 * bw)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s = val(idx + i * bw);
        acc[i] += s * s;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i, idx += bw)
      if (idx < a.n) {
        const float s = val(idx);
        acc[i] += s * s;
      }
  } else {
    for (int64_t i = L; i < a.n; i += bw) {
      const float s = val(i);
      acc[0] += s * s;
    }
  }
  float t = ((acc[0] + acc[1]) + acc[2]) + acc[3];
  __shared__ float part[512];
  __shared__ float total_s;
  if (bw > 64) {
    part[L] = t;
    for (int off = bw / 2; off >= 64; off /= 2) {
      __syncthreads();
      if (L < off) part[L] = t = t + part[L + off];
    }
  }
  if (L < 64) {
    switch (bw) {
      case 1: break;
      case 2: t = group_sum<2>(t); break;
      case 4: t = group_sum<4>(t); break;
      case 8: t = group_sum<8>(t); break;
      case 16: t = group_sum<16>(t); break;
      case 32: t = group_sum<32>(t); break;
      default: t = group_sum<64>(t); break;
    }
    if (L == 0) total_s = t;
  }
  __syncthreads();
  const float rstd = torch_rsqrt(total_s * a.factor + a.eps);
  for (int64_t i = L; i < a.n; i += bw) {
    const float s = val(i);
    if constexpr (ADD) a.res_out[row * a.n + i] = f32_to_bf16(s);  // s read before this (possibly in-place) write
    a.y[row * a.n + i] = f32_to_bf16(round_bf16(s * rstd) * bf16_to_f32(a.w[i]));
  }
}

template <bool ADD, int LANES, int K, bool PART = false>
int launch_fast(const NormArgs& a, hipStream_t s) {
  // the split-K partials' sum (a mixed step's 256 rows of 4 x 4 KB of fp32 each): two rows per 64-thread block, so
  // the rows spread over 4x the CUs (a block streams ~45-50 GB/s): mixed step 2212.6 -> 2169.6 us (one row per
  // 32-thread block 2198 us)
  const int threads = PART ? 2 * LANES : kBlock;
  const int64_t rows_per_block = threads / LANES;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((norm_kernel<LANES, K, ADD, PART>), dim3(unsigned(blocks)), dim3(threads), 0, s, a);
  return check_launch(ADD ? "add_rms_norm" : "rms_norm");
}

// Register-resident kernel when n has one, else the block-per-row kernel. a.factor is set here.
template <bool ADD>
int launch_norm(NormArgs a, bool aligned, hipStream_t s) {
  const int bw = aten_norm_bw(a.n, a.rows);
  a.factor = aten_mean_factor(a.n, a.rows);
  if (aligned && bw > 0) {
    a.m = bw / 64;
    switch (a.n) {
      case 64: return launch_fast<ADD, 8, 1>(a, s);
      case 128: return launch_fast<ADD, 16, 1>(a, s);
      case 256: return launch_fast<ADD, 32, 1>(a, s);
      case 512: return launch_fast<ADD, 32, 2>(a, s);
      case 768: return launch_fast<ADD, 32, 3>(a, s);
      case 1024: return launch_fast<ADD, 32, 4>(a, s);
      case 1536: return launch_fast<ADD, 32, 6>(a, s);
      case 2048: return launch_fast<ADD, 32, 8>(a, s);
      case 2560: return launch_fast<ADD, 32, 10>(a, s);
      case 3072: return launch_fast<ADD, 32, 12>(a, s);
      case 4096: return launch_fast<ADD, 32, 16>(a, s);
      default: break;
    }
  }
  if (a.rows > INT32_MAX) return invalid("rms_norm: too many rows");
  const bool exact = bw > 0 && (a.n < 128 || a.n % 4 == 0);
  a.m = exact ? bw : 0;
  hipLaunchKernelGGL((norm_kernel_generic<ADD>), dim3(unsigned(a.rows)), dim3(exact ? bw : kBlock), 0, s, a);
  return check_launch(ADD ? "add_rms_norm" : "rms_norm");
}

}  // namespace

bool add_rms_norm_partials_supported(int64_t n) { return n == 1024 || n == 2048 || n == 4096; }

int add_rms_norm_partials(uint16_t* y, uint16_t* res_out, const float* xp, int splits, const uint16_t* r,
                          const uint16_t* w, int64_t rows, int64_t n, float eps, hipStream_t s) {
  if (!add_rms_norm_partials_supported(n) || splits < 1 || splits > 4)
    return invalid("add_rms_norm (partials): unsupported size");
  const int bw = aten_norm_bw(n, rows);
  if (bw <= 0) return invalid("add_rms_norm (partials): unsupported size");
  NormArgs a{};
  a.y = y, a.res_out = res_out, a.r = r, a.w = w;
  a.rows = rows, a.r_stride = n, a.n = n, a.eps = eps;
  a.factor = aten_mean_factor(n, rows), a.m = bw / 64;
  a.xp = xp, a.splits = splits, a.xp_split = rows * n;
  switch (n) {
    case 1024: return launch_fast<true, 32, 4, true>(a, s);
    case 2048: return launch_fast<true, 32, 8, true>(a, s);
    default: return launch_fast<true, 32, 16, true>(a, s);
  }
}

}  // namespace nvhip

extern "C" int nvhip_rms_norm_bf16(void* y, const void* x, const void* w, int64_t groups, int64_t rows_per_group,
                                   int64_t group_stride, int64_t row_stride, int64_t n, float eps, void* stream) {
  using namespace nvhip;
  clear_error();
  if (groups < 0 || rows_per_group < 0 || n <= 0) return invalid("rms_norm: bad shape");
  if (group_stride < 0 || row_stride < 0) return invalid("rms_norm: negative stride");
  const int64_t rows = groups * rows_per_group;
  if (rows == 0) return NVHIP_OK;
  if (!y || !x || !w) return invalid("rms_norm: null pointer");
  if (!aligned16(y)) return invalid("rms_norm: y must be 16-byte aligned");
  NormArgs a{};
  a.y = static_cast<uint16_t*>(y);
  a.x = static_cast<const uint16_t*>(x);
  a.w = static_cast<const uint16_t*>(w);
  a.rows = rows, a.rows_per_group = rows_per_group, a.group_stride = group_stride, a.row_stride = row_stride;
  a.n = n, a.eps = eps;
  const bool aligned = aligned16(x) && aligned16(w) && group_stride % 8 == 0 && row_stride % 8 == 0;
  return launch_norm<false>(a, aligned, static_cast<hipStream_t>(stream));
}

extern "C" int nvhip_add_rms_norm_bf16(void* y, void* residual_out, const void* x, const void* residual,
                                       const void* w, int64_t rows, int64_t x_stride, int64_t r_stride, int64_t n,
                                       float eps, void* stream) {
  using namespace nvhip;
  clear_error();
  if (rows < 0 || n <= 0) return invalid("add_rms_norm: bad shape");
  if (x_stride < n || r_stride < n) return invalid("add_rms_norm: row strides must be >= n");
  if (rows == 0) return NVHIP_OK;
  if (!y || !residual_out || !x || !residual || !w) return invalid("add_rms_norm: null pointer");
  if (!aligned16(y) || !aligned16(residual_out)) return invalid("add_rms_norm: outputs must be 16-byte aligned");
  if (residual_out == residual && r_stride != n)
    return invalid("add_rms_norm: in-place residual needs a contiguous residual");
  NormArgs a{};
  a.y = static_cast<uint16_t*>(y);
  a.res_out = static_cast<uint16_t*>(residual_out);
  a.x = static_cast<const uint16_t*>(x);
  a.r = static_cast<const uint16_t*>(residual);
  a.w = static_cast<const uint16_t*>(w);
  a.rows = rows, a.x_stride = x_stride, a.r_stride = r_stride;
  a.n = n, a.eps = eps;
  const bool aligned = aligned16(x) && aligned16(residual) && aligned16(w) && x_stride % 8 == 0 && r_stride % 8 == 0;
  return launch_norm<true>(a, aligned, static_cast<hipStream_t>(stream));
}
