// SiLU x Mul over the [gate | up] halves of a bf16 row, for gfx950.
//
// Replaces nanovllm/kernels/swiglu.py (Triton, :19-43). Numerics of the torch code it stands for
// (layers/activation.py:15-18, F.silu(gate) * up run eagerly):
//   out = bf16(bf16(g / (1 + exp(-g))) * up),   g = fp32(gate)
// with the device expf and a correctly rounded divide, the formula of torch's own silu kernel.
//
// Fast path (n a multiple of 8, 16-byte aligned rows): the [rows, n/8] space of 8-element vectors is flattened;
// a 256-thread block takes VPT runs of 256 consecutive vectors, each thread one vector per run (gate and up are
// two 16-byte loads, the output one 16-byte nontemporal store). The row of a vector comes from a multiply-shift
// division. One vector per thread and plain (not nontemporal) loads: a sweep of 1 / 2 / 4 vectors per thread x
// plain / nontemporal loads (graph replay over 8 rotating inputs) took T = 1 / 32 / 2048 / 8192 (gate_up 6144 wide)
// from 3.12 / 3.28 / 9.26 / 27.17 us (2 vectors, nontemporal) to 2.73 / 3.06 / 8.71 / 26.86 us; 4 vectors per
// thread was the slowest at every T (fewer blocks to spread the latency over).
#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;
constexpr int kVpt = 1;

// n / d and n % d for 0 <= n, d < 2^31 with one mulhi (round-up reciprocal; Granlund & Montgomery 1994, sec. 4).
struct FastDiv {
  uint32_t d, m, s;
  static FastDiv make(uint32_t d) {
    FastDiv f{d, 0, 0};
    while ((1ull << f.s) < d) ++f.s;
    f.m = uint32_t(((1ull << 32) * ((1ull << f.s) - d)) / d + 1);
    return f;
  }
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (__umulhi(n, m) + n) >> s; }
};

struct SiluArgs {
  uint16_t* out;
  const uint16_t* x;
  int64_t x_stride, n;
  uint32_t total;  // rows * n/8 (fast path) or rows * n (generic)
  FastDiv per_row;
};


__global__ __launch_bounds__(kBlock) void silu_mul_kernel(const SiluArgs a) {
  const uint32_t base = blockIdx.x * (kBlock * kVpt) + threadIdx.x;
  u32x4 gate[kVpt], up[kVpt];
  uint32_t row[kVpt], col[kVpt];
#pragma unroll
  for (int k = 0; k < kVpt; ++k) {
    const uint32_t idx = base + k * kBlock;
    row[k] = a.per_row.div(idx);
    col[k] = (idx - row[k] * a.per_row.d) * 8;
    if (idx < a.total) {
      const uint16_t* xr = a.x + int64_t(row[k]) * a.x_stride + col[k];
      gate[k] = load8<true>(xr);
      up[k] = load8<true>(xr + a.n);
    }
  }
#pragma unroll
  for (int k = 0; k < kVpt; ++k) {
    if (base + k * kBlock >= a.total) break;
    float g[8], u[8], o[8];
    unpack8(gate[k], g);
    unpack8(up[k], u);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = silu_bf16(g[i]) * u[i];
    // the output is not read again by this kernel: streamed with the nontemporal hint (~4 % faster at 151 MB)
    __builtin_nontemporal_store(pack8(o), reinterpret_cast<u32x4*>(a.out + int64_t(row[k]) * a.n + col[k]));
  }
}

__global__ __launch_bounds__(kBlock) void silu_mul_kernel_generic(const SiluArgs a) {
  const uint32_t idx = blockIdx.x * kBlock + threadIdx.x;
  if (idx >= a.total) return;
  const uint32_t row = a.per_row.div(idx), col = idx - row * a.per_row.d;
  const uint16_t* xr = a.x + int64_t(row) * a.x_stride + col;
  a.out[int64_t(row) * a.n + col] = f32_to_bf16(silu_bf16(bf16_to_f32(xr[0])) * bf16_to_f32(xr[a.n]));
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_silu_mul_bf16(void* out, const void* x, int64_t rows, int64_t x_stride, int64_t n,
                                   void* stream) {
  using namespace nvhip;
  clear_error();
  if (rows < 0 || n <= 0) return invalid("silu_and_mul: bad shape");
  if (x_stride < 2 * n) return invalid("silu_and_mul: row stride must be >= 2n");
  if (rows == 0) return NVHIP_OK;
  if (!out || !x) return invalid("silu_and_mul: null pointer");
  if (!aligned16(out)) return invalid("silu_and_mul: out must be 16-byte aligned");
  const bool fast = aligned16(x) && n % 8 == 0 && x_stride % 8 == 0;
  const int64_t per_row = fast ? n / 8 : n;
  const int64_t total = rows * per_row;
  if (total >= (int64_t(1) << 31) || per_row >= (int64_t(1) << 31)) return invalid("silu_and_mul: input too large");
  SiluArgs a;
  a.out = static_cast<uint16_t*>(out);
  a.x = static_cast<const uint16_t*>(x);
  a.x_stride = x_stride, a.n = n;
  a.total = uint32_t(total);
  a.per_row = FastDiv::make(uint32_t(per_row));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fast) {
    const int64_t blocks = (total + kBlock * kVpt - 1) / (kBlock * kVpt);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
  } else {
    const int64_t blocks = (total + kBlock - 1) / kBlock;
    hipLaunchKernelGGL(silu_mul_kernel_generic, dim3(unsigned(blocks)), dim3(kBlock), 0, s, a);
  }
  return check_launch("silu_and_mul");
}
