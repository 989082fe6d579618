// GEMM C = A @ B with fp32 accumulation for gfx950.
//
// Replaces nanovllm/kernels/matmul.py (Triton, :11-99): A [M, K], B [K, N] with arbitrary element strides
// (B = W.t() of an nn.Linear weight [N, K] is the common case), fp32 or bf16 inputs, C [M, N] in the input dtype.
// fp32 inputs: precision "ieee" uses them as they are, "tf32" rounds each input to a 10-bit mantissa
// (round to nearest even) before the products, which is what a tf32 tensor-core product sees.
//
// Kernels:
//   gemm_mfma_nt   bf16, A and B both K-contiguous (sak == 1, sbk == 1; B = W.t() of a [N, K] weight):
//                  32x32x16 bf16 MFMA, LDS-staged double-buffered tiles, GROUP_M-swizzled, XCD-aware tile order.
//   gemm_generic   any dtype/strides/precision: 64x64 tile, 4x4 outputs per thread, fp32 FMA.
#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float round_tf32(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;  // inf / nan unchanged
  u += 0xfffu + ((u >> 13) & 1u);
  return __uint_as_float(u & 0xffffe000u);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

struct GemmArgs {
  void* c;
  const void* a;
  const void* b;
  int64_t M, N, K;
  int64_t sam, sak, sbk, sbn, scm, scn;
};

// 64x64 output tile per 256-thread block; thread (ty, tx) owns rows ty + 16*i, cols tx + 16*j (i, j < 4).
// K is staged 16 at a time through LDS; out-of-range elements load as 0.
template <typename T, bool TF32>
__global__ __launch_bounds__(kBlock) void gemm_generic(const GemmArgs g) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float As[BK][BM + 1];
  __shared__ float Bs[BK][BN + 1];
  const T* A = static_cast<const T*>(g.a);
  const T* B = static_cast<const T*>(g.b);
  T* C = static_cast<T*>(g.c);
  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < g.K; k0 += BK) {
    for (int i = threadIdx.x; i < BM * BK; i += kBlock) {
      const int r = i / BK, kk = i % BK;
      const int64_t m = m0 + r, k = k0 + kk;
      float v = (m < g.M && k < g.K) ? to_f32<T>(A[m * g.sam + k * g.sak]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      As[kk][r] = v;
    }
    for (int i = threadIdx.x; i < BN * BK; i += kBlock) {
      const int cidx = i % BN, kk = i / BN;
      const int64_t n = n0 + cidx, k = k0 + kk;
      float v = (n < g.N && k < g.K) ? to_f32<T>(B[k * g.sbk + n * g.sbn]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      Bs[kk][cidx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
      if (m < g.M && n < g.N) C[m * g.scm + n * g.scn] = from_f32<T>(acc[i][j]);
    }
}


// ------------------------------------------------------------------------------------------------------------
// bf16 MFMA kernel (A and B K-contiguous, C row-major with unit column stride).
//
// Block tile BM x BN x 64, 256 threads = 4 waves in a WAVES_M x WAVES_N grid, each wave owning WM x WN outputs
// as FM x FN tiles of v_mfma_f32_32x32x16_bf16. The MFMA is issued with the operands swapped (its "A" is the
// B^T = W fragment, its "B" the A fragment), so a lane's 16 accumulators hold, for one output row m, four runs of
// 4 consecutive columns: the epilogue stores 8 bytes per lane per run.
//   lane l, accumulator r of tile (fm, fn):  m = fm*32 + l%32,  n = fn*32 + 8*(r/4) + 4*(l/32) + r%4
// Operand fragments (verified on gfx950): lane l reads row l%32, k = 8*(l/32) .. +8 of the 16-wide k step.
//
// LDS: A and B tiles [rows][64] bf16 (128 bytes a row, eight 16-byte chunks), chunk c of row r stored at chunk
// position c ^ (r & 7) so that the 32 rows a fragment read touches spread over all banks. Two stages: the global
// loads of k-tile kt+1 are in flight (in registers) while k-tile kt is multiplied, then written to the other
// stage; one barrier per k-tile.
//
// Tile order: 1-D grid; the block id is first remapped so that consecutive ids run on the same XCD (the dispatcher
// deals blocks round-robin over the 8 XCDs), then mapped through the GROUP_M swizzle of the reference
// (matmul.py:50-57): tile-rows in groups of GROUP_M, column-major inside a group, so blocks that run together
// share A rows and B columns in their XCD's L2.
// Rows past M / columns past N are loaded clamped to the last row (and never stored); k past K loads as zero.
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kGroupM = 8;
constexpr int kBK = 64;

struct MfmaArgs {
  uint16_t* c;
  const uint16_t* a;
  const uint16_t* w;  // B^T: element (n, k) at w + n*swn + k
  int M, N, K;
  int64_t sam, swn, scm;
};

__device__ __forceinline__ void tile_coords(int pid, int M, int N, int BM, int BN, int& pid_m, int& pid_n) {
  const int num_m = (M + BM - 1) / BM, num_n = (N + BN - 1) / BN;
  const int total = num_m * num_n;
  if (total % 8 == 0) {
    const int per_xcd = total / 8;
    pid = (pid % 8) * per_xcd + pid / 8;
  }
  const int in_group = kGroupM * num_n;
  const int first_m = (pid / in_group) * kGroupM;
  const int group_rows = min(num_m - first_m, kGroupM);
  pid_m = first_m + (pid % in_group) % group_rows;
  pid_n = (pid % in_group) / group_rows;
}

template <int BM, int BN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(256) void gemm_mfma_nt(const MfmaArgs g) {
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int FM = WM / 32, FN = WN / 32;
  static_assert(WAVES_M * WAVES_N == 4 && FM >= 1 && FN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  constexpr int A_CHUNKS = BM * 8 / 256, B_CHUNKS = BN * 8 / 256;  // 16-byte chunks per thread per k-tile
  static_assert(A_CHUNKS >= 1 && B_CHUNKS >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * kBK];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * kBK];

  int pid_m, pid_n;
  tile_coords(blockIdx.x, g.M, g.N, BM, BN, pid_m, pid_n);
  const int m0 = pid_m * BM, n0 = pid_n * BN;
  const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // global -> register staging: thread tid loads chunks tid + 256*i (row = chunk / 8, k-chunk = chunk % 8)
  const uint16_t* a_src[A_CHUNKS];
  const uint16_t* b_src[B_CHUNKS];
  int a_lds[A_CHUNKS], b_lds[B_CHUNKS], a_kc[A_CHUNKS], b_kc[B_CHUNKS];
#pragma unroll
  for (int i = 0; i < A_CHUNKS; ++i) {
    const int ch = tid + 256 * i, row = ch / 8, kc = ch % 8;
    a_src[i] = g.a + int64_t(min(m0 + row, g.M - 1)) * g.sam + kc * 8;
    a_lds[i] = row * kBK + ((kc ^ (row & 7)) * 8);
    a_kc[i] = kc * 8;
  }
#pragma unroll
  for (int i = 0; i < B_CHUNKS; ++i) {
    const int ch = tid + 256 * i, row = ch / 8, kc = ch % 8;
    b_src[i] = g.w + int64_t(min(n0 + row, g.N - 1)) * g.swn + kc * 8;
    b_lds[i] = row * kBK + ((kc ^ (row & 7)) * 8);
    b_kc[i] = kc * 8;
  }
  u32x4 ra[A_CHUNKS], rb[B_CHUNKS];
  auto load_tile = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i)
      ra[i] = (k0 + a_kc[i] < g.K) ? *reinterpret_cast<const u32x4*>(a_src[i] + k0) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i)
      rb[i] = (k0 + b_kc[i] < g.K) ? *reinterpret_cast<const u32x4*>(b_src[i] + k0) : u32x4{0, 0, 0, 0};
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CHUNKS; ++i) *reinterpret_cast<u32x4*>(&As[buf][a_lds[i]]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CHUNKS; ++i) *reinterpret_cast<u32x4*>(&Bs[buf][b_lds[i]]) = rb[i];
  };

  f32x16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16_t{};

  // fragment read offsets: row = base + l%32 (row & 7 == l & 7), chunk = 2*kk + l/32
  const int frag_row = lane % 32, frag_half = lane / 32, swz = lane & 7;
  const int nk = (g.K + kBK - 1) / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_tile((kt + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int chunk = ((2 * kk + frag_half) ^ swz) * 8;
      bf16x8_t af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_t*>(&As[buf][(wm * WM + i * 32 + frag_row) * kBK + chunk]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][(wn * WN + j * 32 + frag_row) * kBK + chunk]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds row m, columns n .. n+3 for each run
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    const int m = m0 + wm * WM + i * 32 + frag_row;
    if (m >= g.M) continue;
    uint16_t* crow = g.c + int64_t(m) * g.scm;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int run = 0; run < 4; ++run) {
        const int n = n0 + wn * WN + j * 32 + 8 * run + 4 * frag_half;
        const float v0 = acc[i][j][4 * run], v1 = acc[i][j][4 * run + 1];
        const float v2 = acc[i][j][4 * run + 2], v3 = acc[i][j][4 * run + 3];
        if (n + 3 < g.N) {
          typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
          *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
        } else {
          const float v[4] = {v0, v1, v2, v3};
          for (int e = 0; e < 4 && n + e < g.N; ++e) crow[n + e] = f32_to_bf16(v[e]);
        }
      }
  }
}

template <int BM, int BN, int WAVES_M, int WAVES_N>
int launch_mfma(const MfmaArgs& g, hipStream_t s) {
  const int64_t tiles = int64_t((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  hipLaunchKernelGGL((gemm_mfma_nt<BM, BN, WAVES_M, WAVES_N>), dim3(unsigned(tiles)), dim3(256), 0, s, g);
  return check_launch("matmul");
}

// Tile shape for an M x N output: enough tiles to fill the 256 CUs at the largest tile that allows it.
int launch_mfma_auto(const MfmaArgs& g, hipStream_t s) {
  auto tiles = [&](int bm, int bn) { return int64_t((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn); };
  if (g.M <= 32) return launch_mfma<32, 128, 1, 4>(g, s);
  if (g.M <= 64) return launch_mfma<64, 128, 2, 2>(g, s);
  if (tiles(256, 128) >= 256) return launch_mfma<256, 128, 2, 2>(g, s);
  if (tiles(128, 128) >= 256) return launch_mfma<128, 128, 2, 2>(g, s);
  return launch_mfma<128, 64, 2, 2>(g, s);
}

template <typename T, bool TF32>
int launch_generic(const GemmArgs& g, hipStream_t s) {
  const int64_t gx = (g.N + 63) / 64, gy = (g.M + 63) / 64;
  if (gx > INT32_MAX || gy > 65535) return invalid("matmul: matrix too large");
  hipLaunchKernelGGL((gemm_generic<T, TF32>), dim3(unsigned(gx), unsigned(gy)), dim3(kBlock), 0, s, g);
  return check_launch("matmul");
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_matmul(void* c, const void* a, const void* b, int64_t M, int64_t N, int64_t K, int64_t sam,
                            int64_t sak, int64_t sbk, int64_t sbn, int64_t scm, int64_t scn, int dtype,
                            int precision, void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N < 0 || K < 0) return invalid("matmul: negative size");
  if (sam < 0 || sak < 0 || sbk < 0 || sbn < 0 || scm < 0 || scn < 0) return invalid("matmul: negative stride");
  if (dtype != NVHIP_DTYPE_F32 && dtype != NVHIP_DTYPE_BF16) return invalid("matmul: dtype must be fp32 or bf16");
  if (precision != NVHIP_PREC_IEEE && precision != NVHIP_PREC_TF32)
    return invalid("matmul: precision must be ieee or tf32");
  if (M == 0 || N == 0) return NVHIP_OK;
  if (!c || (K > 0 && (!a || !b))) return invalid("matmul: null pointer");
  GemmArgs g{c, a, b, M, N, K, sam, sak, sbk, sbn, scm, scn};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NVHIP_DTYPE_BF16) {
    // MFMA path: A and B K-contiguous with 16-byte aligned rows, C with unit column stride, sizes within int32
    const bool nt = sak == 1 && sbk == 1 && scn == 1 && K % 8 == 0 && K > 0 && sam % 8 == 0 && sbn % 8 == 0 &&
                    aligned16(a) && aligned16(b) && (reinterpret_cast<uintptr_t>(c) & 7) == 0 && scm % 4 == 0 &&
                    M < (int64_t(1) << 31) && N < (int64_t(1) << 31) && K < (int64_t(1) << 31);
    if (nt) {
      MfmaArgs m{static_cast<uint16_t*>(c), static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b),
                 int(M), int(N), int(K), sam, sbn, scm};
      return launch_mfma_auto(m, s);
    }
    return launch_generic<uint16_t, false>(g, s);
  }
  if (precision == NVHIP_PREC_TF32) return launch_generic<float, true>(g, s);
  return launch_generic<float, false>(g, s);
}
