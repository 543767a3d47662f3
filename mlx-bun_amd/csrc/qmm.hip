// qmm.hip -- mx.quantized_matmul for MLX affine-quantized weights (gfx950).
//
// Main path (transpose = true, bits in {4, 8}, group 64/128, T = bf16/f16):
// the weight stream is the roofline, so codes never leave registers as
// anything but exact MFMA operands.  Per 64-k tile (one quantization group
// for gs = 64) each lane loads the 16 codes of one weight row it owns, turns
// them into two k-steps of a v_mfma_f32_16x16x32 B operand by the
// mantissa-OR trick (mfma_common.h), and the group's
//     y += s * sum_k x_k (c_k + off)  +  (b - off * s) * sum_k x_k
// is applied to the 16x16 accumulator once per group.  sum_k x_k comes from a
// second MFMA against a ones operand, so no VALU work depends on M.
// x operands are read from global memory (L1/L2 resident; identical
// addresses across lanes when M is small) and permuted into the codes' slot
// order in registers.  Work: a workgroup = 16 weight rows; its waves split K
// and reduce in LDS (deterministic, no cross-workgroup traffic).
//
// Everything else (transpose = false, 2-bit, group 32, fp32 activations,
// odd shapes) takes a straightforward VALU kernel.
#include "mfma_common.h"

namespace {

constexpr int QMV_CT = 8;  // tiles per register chunk (double-buffered)

// Load one chunk of QMV_CT 64-k tiles of this lane's weight row (16 codes per
// tile) plus their scales/biases.
template <typename T, int BITS, int GS>
__device__ __forceinline__ void qmv_load_chunk(const uint32_t* __restrict__ wrow_ptr, const uint16_t* __restrict__ srow,
                                               const uint16_t* __restrict__ brow, int tile0, int tile_end, int lg,
                                               uint32_t (&wreg)[QMV_CT][BITS / 2], float (&sreg)[QMV_CT],
                                               float (&breg)[QMV_CT]) {
  constexpr int WPT = BITS / 2;
#pragma unroll
  for (int t = 0; t < QMV_CT; t++) {
    const int tile = tile0 + t;
    if (tile < tile_end) {
      const uint32_t* src = wrow_ptr + ((int64_t)tile * 64 + lg * 16) * BITS / 32;
      if constexpr (WPT == 2) {
        const uint2 v = *reinterpret_cast<const uint2*>(src);
        wreg[t][0] = v.x;
        wreg[t][WPT - 1] = v.y;
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(src);
        wreg[t][0] = v.x;
        wreg[t][1 % WPT] = v.y;
        wreg[t][2 % WPT] = v.z;
        wreg[t][3 % WPT] = v.w;
      }
      sreg[t] = Conv<T>::from_bits(srow[(int64_t)tile * 64 / GS]);
      breg[t] = Conv<T>::from_bits(brow[(int64_t)tile * 64 / GS]);
    }
  }
}

template <typename T, int BITS, int GS, int MB>
__device__ __forceinline__ void qmv_compute_chunk(const uint16_t* __restrict__ x, int64_t M, int64_t K, int tile0,
                                                  int tile_end, int ln, int lg,
                                                  const uint32_t (&wreg)[QMV_CT][BITS / 2],
                                                  const float (&sreg)[QMV_CT], const float (&breg)[QMV_CT],
                                                  f32x4_t (&yacc)[MB]) {
  using CO = CodeOps<T, BITS>;
  constexpr int WPT = BITS / 2;
  const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};
#pragma unroll
  for (int t = 0; t < QMV_CT; t++) {
    const int tile = tile0 + t;
    if (tile < tile_end) {
      u32x4_t b0, b1;
      if constexpr (BITS == 4) {
        b0 = CodeOps<T, 4>::operand(wreg[t][0]);
        b1 = CodeOps<T, 4>::operand(wreg[t][WPT - 1]);
      } else {
        b0 = CodeOps<T, BITS>::operand(wreg[t][0], wreg[t][1 % WPT]);
        b1 = CodeOps<T, BITS>::operand(wreg[t][2 % WPT], wreg[t][3 % WPT]);
      }
      const float sc = sreg[t];
      const float bb = breg[t] - CO::OFFSET * sc;
      const int64_t k = (int64_t)tile * 64 + lg * 16;
#pragma unroll
      for (int rb = 0; rb < MB; rb++) {
        int64_t m = rb * 16 + ln;
        m = m < M ? m : M - 1;
        const uint16_t* xr = x + m * K + k;
        const u32x4_t a0 = permute8<CO::ORDER>(*reinterpret_cast<const u32x4_t*>(xr));
        const u32x4_t a1 = permute8<CO::ORDER>(*reinterpret_cast<const u32x4_t*>(xr + 8));
        // D = x (A, rows m) . codes (B, cols n); the ones operand gives sum x
        f32x4_t acc = Mma<T>::mma(a0, b0, f32x4_t{0.f, 0.f, 0.f, 0.f});
        acc = Mma<T>::mma(a1, b1, acc);
        f32x4_t xs = Mma<T>::mma(a0, ones, f32x4_t{0.f, 0.f, 0.f, 0.f});
        xs = Mma<T>::mma(a1, ones, xs);
#pragma unroll
        for (int i = 0; i < 4; i++) yacc[rb][i] += sc * acc[i] + bb * xs[i];
      }
    }
  }
}

// One workgroup = 16 weight rows (MFMA columns); its NW waves split the K
// axis into contiguous tile ranges and their partial sums meet in LDS.  No
// cross-workgroup traffic.  Weight codes are double-buffered in registers
// by chunks of QMV_CT tiles so the next chunk's loads are in flight while
// the current one computes.
template <typename T, int BITS, int GS, int MB, int NW>
__global__ void __launch_bounds__(NW * 64) qmv_mfma_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                            const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ biases, int64_t N,
                                                            int64_t w_rep, uint16_t* __restrict__ y) {
  constexpr int WPT = BITS / 2;
  __shared__ f32x4_t red[NW][MB][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int64_t bidx = blockIdx.y;
  const int64_t wb = bidx / w_rep;
  x += bidx * M * K;
  y += bidx * M * N;
  w += wb * N * (K * BITS / 32);
  scales += wb * N * (K / GS);
  biases += wb * N * (K / GS);

  const int64_t n = (int64_t)blockIdx.x * 16 + ln;
  const int64_t nl = n < N ? n : N - 1;  // clamp loads; stores are masked
  const int tiles = (int)(K / 64);
  const int per = (tiles + NW - 1) / NW;
  const int t_begin = min(tiles, wave * per);
  const int t_end = min(tiles, t_begin + per);
  const uint32_t* wrow_ptr = w + nl * (K * BITS / 32);
  const uint16_t* srow = scales + nl * (K / GS);
  const uint16_t* brow = biases + nl * (K / GS);

  f32x4_t yacc[MB];
#pragma unroll
  for (int rb = 0; rb < MB; rb++) yacc[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t wa[QMV_CT][WPT], wbuf[QMV_CT][WPT];
  float sa[QMV_CT], ba[QMV_CT], sb2[QMV_CT], bb2[QMV_CT];
  qmv_load_chunk<T, BITS, GS>(wrow_ptr, srow, brow, t_begin, t_end, lg, wa, sa, ba);
  for (int c0 = t_begin; c0 < t_end; c0 += 2 * QMV_CT) {
    const int c1 = c0 + QMV_CT;
    if (c1 < t_end) qmv_load_chunk<T, BITS, GS>(wrow_ptr, srow, brow, c1, t_end, lg, wbuf, sb2, bb2);
    qmv_compute_chunk<T, BITS, GS, MB>(x, M, K, c0, t_end, ln, lg, wa, sa, ba, yacc);
    if (c1 < t_end) {
      if (c1 + QMV_CT < t_end) qmv_load_chunk<T, BITS, GS>(wrow_ptr, srow, brow, c1 + QMV_CT, t_end, lg, wa, sa, ba);
      qmv_compute_chunk<T, BITS, GS, MB>(x, M, K, c1, t_end, ln, lg, wbuf, sb2, bb2, yacc);
    }
  }

  // ---- reduce the NW waves' partials; D layout row = 4*lg + i, col = ln ---
#pragma unroll
  for (int rb = 0; rb < MB; rb++) red[wave][rb][lane] = yacc[rb];
  __syncthreads();
  if (wave == 0 && n < N) {
#pragma unroll
    for (int rb = 0; rb < MB; rb++) {
      f32x4_t acc = red[0][rb][lane];
#pragma unroll
      for (int wv = 1; wv < NW; wv++) {
        const f32x4_t o = red[wv][rb][lane];
        acc[0] += o[0];
        acc[1] += o[1];
        acc[2] += o[2];
        acc[3] += o[3];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t m = rb * 16 + lg * 4 + i;
        if (m < M) y[m * N + n] = (uint16_t)Conv<T>::to_bits(acc[i]);
      }
    }
  }
}

// ---- generic VALU path -----------------------------------------------------
// One thread per output element; fp32 accumulation of fp32-dequantized
// weights.  transpose=1: W [N, K] grouped along K.  transpose=0: W [K, N]
// grouped along N.
template <typename T, int BITS>
__global__ void __launch_bounds__(256) qmm_generic_kernel(const void* __restrict__ xv, int64_t M, int64_t K,
                                                           const uint32_t* __restrict__ w, const void* __restrict__ sv,
                                                           const void* __restrict__ bv, int64_t N, int gs,
                                                           int transpose, int64_t w_rep, void* __restrict__ yv) {
  using S = typename T::storage;
  const S* x = reinterpret_cast<const S*>(xv);
  const S* scales = reinterpret_cast<const S*>(sv);
  const S* biases = reinterpret_cast<const S*>(bv);
  S* y = reinterpret_cast<S*>(yv);
  const int64_t bidx = blockIdx.z;
  const int64_t wb = bidx / w_rep;
  const int64_t mn = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (mn >= M * N) return;
  const int64_t m = mn / N, n = mn % N;
  x += bidx * M * K;
  y += bidx * M * N;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  constexpr int E = 32 / BITS;
  float acc = 0.f;
  if (transpose) {
    const int64_t wrow = K / E, grow = K / gs;
    const uint32_t* wr = w + (wb * N + n) * wrow;
    const S* sr = scales + (wb * N + n) * grow;
    const S* br = biases + (wb * N + n) * grow;
    for (int64_t k = 0; k < K; k++) {
      const float c = (float)((wr[k / E] >> (BITS * (k % E))) & MASK);
      const float wv = Conv<T>::load(sr, k / gs) * c + Conv<T>::load(br, k / gs);
      acc += Conv<T>::load(x, m * K + k) * wv;
    }
  } else {
    const int64_t wrow = N / E, grow = N / gs;
    for (int64_t k = 0; k < K; k++) {
      const int64_t r = wb * K + k;
      const float c = (float)((w[r * wrow + n / E] >> (BITS * (n % E))) & MASK);
      const float wv = Conv<T>::load(scales, r * grow + n / gs) * c + Conv<T>::load(biases, r * grow + n / gs);
      acc += Conv<T>::load(x, m * K + k) * wv;
    }
  }
  Conv<T>::store(y, m * N + n, acc);
}

template <typename T, int BITS, int GS, int MB>
int launch_qmv_mb(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                  const void* biases, int64_t w_rep, int64_t N, void* y, hipStream_t s) {
  // waves per workgroup: enough for ~8 waves per CU over the launch, capped
  // so the LDS reduction (NW * MB KiB) stays small
  const int64_t groups = (N + 15) / 16 * batch;
  const int64_t want_waves = (int64_t)mlxq::device_cu_count() * 8;
  int nw = 1;
  while (nw < 8 && groups * nw < want_waves && (K / 64) / (2 * nw) >= 2) nw *= 2;
  dim3 grid((unsigned)((N + 15) / 16), (unsigned)batch);
#define QMV_LAUNCH(NWV)                                                                                      \
  hipLaunchKernelGGL((qmv_mfma_kernel<T, BITS, GS, MB, NWV>), grid, dim3(NWV * 64), 0, s, (const uint16_t*)x, M, K, \
                     w, (const uint16_t*)scales, (const uint16_t*)biases, N, w_rep, (uint16_t*)y)
  switch (nw) {
    case 1: QMV_LAUNCH(1); break;
    case 2: QMV_LAUNCH(2); break;
    case 4: QMV_LAUNCH(4); break;
    default: QMV_LAUNCH(8); break;
  }
#undef QMV_LAUNCH
  MLXQ_LAUNCHED("qmv_mfma_kernel");
  return MLXQ_OK;
}

template <typename T, int BITS, int GS>
int launch_qmv(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
               const void* biases, int64_t w_rep, int64_t N, void* y, hipStream_t s) {
  switch ((M + 15) / 16) {
    case 1: return launch_qmv_mb<T, BITS, GS, 1>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    case 2: return launch_qmv_mb<T, BITS, GS, 2>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    case 3: return launch_qmv_mb<T, BITS, GS, 3>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    case 4: return launch_qmv_mb<T, BITS, GS, 4>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    default: return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: M > 64");
  }
}

}  // namespace

extern "C" int mlxq_quantized_matmul(const void* x, int dtype, int64_t batch, int64_t M, int64_t K,
                                     const uint32_t* w, const void* scales, const void* biases, int64_t w_batch,
                                     int64_t N, int group_size, int bits, int transpose, void* y, void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_CHECK(mlxq::dtype_supported(dtype), "dtype must be float16, bfloat16 or float32");
  MLXQ_CHECK(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");
  MLXQ_CHECK(group_size == 32 || group_size == 64 || group_size == 128, "group_size must be 32, 64 or 128");
  MLXQ_CHECK(batch >= 0 && M >= 0 && K >= 0 && N >= 0, "negative extent");
  MLXQ_CHECK(w_batch >= 1 && batch % w_batch == 0, "batch must be a multiple of w_batch");
  const int64_t grouped = transpose ? K : N;
  MLXQ_CHECK(grouped % group_size == 0, "the quantized axis must be a multiple of group_size");
  if (batch == 0 || M == 0 || N == 0) return MLXQ_OK;
  MLXQ_CHECK(x && w && scales && biases && y, "null buffer");
  hipStream_t s = mlxq::resolve_stream(stream);
  const int64_t w_rep = batch / w_batch;
  if (K == 0) return mlxq_fill_zero(y, (uint64_t)(batch * M * N * mlxq::dtype_bytes(dtype)), stream);

  const bool mfma_ok = transpose && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                       (group_size == 64 || group_size == 128) && K % 64 == 0 && M <= 64 &&
                       (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0;
  if (mfma_ok) {
    if (dtype == MLXQ_BFLOAT16) {
      if (bits == 4)
        return group_size == 64 ? launch_qmv<BF16, 4, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s)
                                : launch_qmv<BF16, 4, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
      return group_size == 64 ? launch_qmv<BF16, 8, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s)
                              : launch_qmv<BF16, 8, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    } else {
      if (bits == 4)
        return group_size == 64 ? launch_qmv<F16, 4, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s)
                                : launch_qmv<F16, 4, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
      return group_size == 64 ? launch_qmv<F16, 8, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s)
                              : launch_qmv<F16, 8, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);
    }
  }

  const int64_t outs = M * N;
  MLXQ_CHECK(outs <= (int64_t)0x7fffffff * 256, "output too large");
  dim3 grid((unsigned)((outs + 255) / 256), 1, (unsigned)batch);
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 2>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, w_rep, y);
        break;
      case 4:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 4>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, w_rep, y);
        break;
      default:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 8>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, w_rep, y);
        break;
    }
  });
  MLXQ_LAUNCHED("qmm_generic_kernel");
  return MLXQ_OK;
}
