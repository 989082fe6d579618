// RMSNorm and Add+RMSNorm over bf16 rows, for gfx950.
//
// Replace nanovllm/kernels/rms_norm.py (Triton, :34-111). Numerics of the torch code they stand for
// (layers/layernorm.py:20-44):
//   rms_norm:      y = bf16(bf16(x * rstd) * w),             rstd = 1 / sqrt(sum(x^2) * (1/n) + eps)
//   add_rms_norm:  s = fp32(x) + fp32(r); res = bf16(s);    y = bf16(bf16(s * rstd) * w), rstd from the fp32 s
// sqrt and the divide are correctly rounded; only the order of the fp32 sum of squares differs from torch.
//
// Fast path (n a multiple of 8 with 16-byte aligned rows, n/8 = LANES * VPL): LANES consecutive lanes of a wave64
// own a row, each holding VPL 16-byte vectors (vector j of lane l = elements [(j*LANES + l)*8, +8), so a wave's
// loads are contiguous), the row stays in registers between the reduction and the output, and the sum of squares
// is a LANES-wide DPP/shuffle reduction. Other shapes use a block-per-row fallback.
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
  float inv_n, eps;
  // add_rms_norm with x given as splits (1..4) fp32 partial products [splits, rows, n] (split s at xp + s * xp_split):
  // x = bf16(sum of the partials in split order), the rounding of the GEMM output they add up to
  const float* xp;
  int splits;
  int64_t xp_split;
};

template <int LANES, int VPL, bool ADD, bool PART = false>
__global__ __launch_bounds__(kBlock) void norm_kernel(const NormArgs a) {
  constexpr int N = LANES * VPL * 8;
  const int sub = threadIdx.x % LANES;
  const int64_t row = int64_t(blockIdx.x) * (kBlock / LANES) + threadIdx.x / LANES;
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

  float v[VPL][8];
  u32x4 raw[VPL], wraw[VPL];
  if constexpr (PART) {  // every split's vectors loaded at once, then summed in split order and rounded to bf16
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const float* xp = a.xp + row * a.n;
    f32x4 p[4][VPL][2];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (s < a.splits)
#pragma unroll
        for (int j = 0; j < VPL; ++j)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            p[s][j][h] = *reinterpret_cast<const f32x4*>(xp + s * a.xp_split + (j * LANES + sub) * 8 + 4 * h);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float x[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = p[0][j][i / 4][i % 4];
#pragma unroll
      for (int s = 1; s < 4; ++s)
        if (s < a.splits)
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] += p[s][j][i / 4][i % 4];
      raw[j] = pack8(x);
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) raw[j] = load8<true>(xr + (j * LANES + sub) * 8);
  }
  // the weight is loaded up front: after the residual store the compiler could not move it past a possible alias
#pragma unroll
  for (int j = 0; j < VPL; ++j) wraw[j] = load8<true>(a.w + (j * LANES + sub) * 8);
  if constexpr (ADD) {
    u32x4 rraw[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) rraw[j] = load8<true>(rr + (j * LANES + sub) * 8);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      float xf[8], rf[8];
      unpack8(raw[j], xf);
      unpack8(rraw[j], rf);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[j][i] = xf[i] + rf[i];
      store8<true>(a.res_out + row * N + (j * LANES + sub) * 8, pack8(v[j]));
    }
  } else {
#pragma unroll
    for (int j = 0; j < VPL; ++j) unpack8(raw[j], v[j]);
  }

  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < VPL; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
  ss = group_sum<LANES>(ss);
  const float rstd = 1.0f / sqrtf(ss * a.inv_n + a.eps);

#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    float wf[8], o[8];
    unpack8(wraw[j], wf);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = round_bf16(v[j][i] * rstd) * wf[i];
    uint16_t* dst = a.y + row * N + (j * LANES + sub) * 8;
    // plain RMSNorm streams its output (measured faster); Add+RMSNorm keeps plain stores (measured slower with the
    // hint on either output)
    if constexpr (ADD) store8<true>(dst, pack8(o));
    else __builtin_nontemporal_store(pack8(o), reinterpret_cast<u32x4*>(dst));
  }
}

// Fallback: one block per row, any n and alignment. Two passes over the row (the second mostly hits the cache).
template <bool ADD>
__global__ __launch_bounds__(kBlock) void norm_kernel_generic(const NormArgs a) {
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
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < a.n; i += kBlock) {
    float s = bf16_to_f32(xr[i]);
    if constexpr (ADD) s += bf16_to_f32(rr[i]);
    ss += s * s;
  }
  __shared__ float partial[kBlock / 64];
  ss = group_sum<64>(ss);
  if (threadIdx.x % 64 == 0) partial[threadIdx.x / 64] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kBlock / 64; ++i) total += partial[i];
  const float rstd = 1.0f / sqrtf(total * a.inv_n + a.eps);
  for (int64_t i = threadIdx.x; i < a.n; i += kBlock) {
    float s = bf16_to_f32(xr[i]);
    if constexpr (ADD) {
      s += bf16_to_f32(rr[i]);  // read before the (possibly in-place) residual write below
      a.res_out[row * a.n + i] = f32_to_bf16(s);
    }
    a.y[row * a.n + i] = f32_to_bf16(round_bf16(s * rstd) * bf16_to_f32(a.w[i]));
  }
}

template <bool ADD, int LANES, int VPL, bool PART = false>
int launch_fast(const NormArgs& a, hipStream_t s) {
  const int64_t rows_per_block = kBlock / LANES;
  const int64_t blocks = (a.rows + rows_per_block - 1) / rows_per_block;
  hipLaunchKernelGGL((norm_kernel<LANES, VPL, ADD, PART>), dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
  return check_launch(ADD ? "add_rms_norm" : "rms_norm");
}

// Register-resident kernel when n has one, else the block-per-row fallback.
template <bool ADD>
int launch_norm(const NormArgs& a, bool aligned, hipStream_t s) {
  if (aligned && a.n % 8 == 0) {
    switch (a.n / 8) {
      case 8: return launch_fast<ADD, 8, 1>(a, s);     // n = 64
      case 16: return launch_fast<ADD, 16, 1>(a, s);   // n = 128
      case 32: return launch_fast<ADD, 32, 1>(a, s);   // n = 256
      case 64: return launch_fast<ADD, 64, 1>(a, s);   // n = 512
      case 128: return launch_fast<ADD, 64, 2>(a, s);  // n = 1024
      case 192: return launch_fast<ADD, 64, 3>(a, s);  // n = 1536
      case 256: return launch_fast<ADD, 64, 4>(a, s);  // n = 2048
      case 320: return launch_fast<ADD, 64, 5>(a, s);  // n = 2560
      case 384: return launch_fast<ADD, 64, 6>(a, s);  // n = 3072
      case 512: return launch_fast<ADD, 64, 8>(a, s);  // n = 4096
      case 640: return launch_fast<ADD, 64, 10>(a, s); // n = 5120
      case 768: return launch_fast<ADD, 64, 12>(a, s); // n = 6144
      case 1024: return launch_fast<ADD, 64, 16>(a, s); // n = 8192
      default: break;
    }
  }
  if (a.rows > INT32_MAX) return invalid("rms_norm: too many rows");
  hipLaunchKernelGGL((norm_kernel_generic<ADD>), dim3(unsigned(a.rows)), dim3(kBlock), 0, s, a);
  return check_launch(ADD ? "add_rms_norm" : "rms_norm");
}

}  // namespace

bool add_rms_norm_partials_supported(int64_t n) { return n == 1024 || n == 2048 || n == 4096; }

int add_rms_norm_partials(uint16_t* y, uint16_t* res_out, const float* xp, int splits, const uint16_t* r,
                          const uint16_t* w, int64_t rows, int64_t n, float eps, hipStream_t s) {
  if (!add_rms_norm_partials_supported(n) || splits < 1 || splits > 4)
    return invalid("add_rms_norm (partials): unsupported size");
  NormArgs a{};
  a.y = y, a.res_out = res_out, a.r = r, a.w = w;
  a.rows = rows, a.r_stride = n, a.n = n, a.inv_n = 1.0f / float(n), a.eps = eps;
  a.xp = xp, a.splits = splits, a.xp_split = rows * n;
  switch (n) {
    case 1024: return launch_fast<true, 64, 2, true>(a, s);
    case 2048: return launch_fast<true, 64, 4, true>(a, s);
    default: return launch_fast<true, 64, 8, true>(a, s);
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
  a.n = n, a.inv_n = 1.0f / float(n), a.eps = eps;
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
  a.n = n, a.inv_n = 1.0f / float(n), a.eps = eps;
  const bool aligned = aligned16(x) && aligned16(residual) && aligned16(w) && x_stride % 8 == 0 && r_stride % 8 == 0;
  return launch_norm<true>(a, aligned, static_cast<hipStream_t>(stream));
}
