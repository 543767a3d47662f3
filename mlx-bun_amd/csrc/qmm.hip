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
// x is staged once per workgroup in LDS, already permuted into the slot
// order of the code operands.  Work: a workgroup = 4 waves x 16 weight rows,
// the K axis optionally split over `ks` workgroups whose fp32 partials the
// last-arriving workgroup sums in fixed order (deterministic).
//
// Everything else (transpose = false, 2-bit, group 32, fp32 activations,
// odd shapes) takes a straightforward VALU kernel.
#include "mfma_common.h"

namespace {

constexpr int QMV_WAVES = 4;
constexpr int QMV_COLS = 16 * QMV_WAVES;  // weight rows per workgroup
constexpr int QMV_MAXT = 16;              // 64-k tiles per wave per split

template <typename T, int BITS, int GS, int MB>
__global__ void __launch_bounds__(256) qmv_mfma_kernel(const uint16_t* __restrict__ x, int64_t M, int64_t K,
                                                        const uint32_t* __restrict__ w,
                                                        const uint16_t* __restrict__ scales,
                                                        const uint16_t* __restrict__ biases, int64_t N,
                                                        int64_t w_rep, int64_t k_split, uint16_t* __restrict__ y,
                                                        float* __restrict__ partial, uint32_t* __restrict__ counters) {
  using CO = CodeOps<T, BITS>;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ks = blockIdx.y;
  const int nks = gridDim.y;
  const int64_t bidx = blockIdx.z;
  const int64_t wb = bidx / w_rep;
  x += bidx * M * K;
  y += bidx * M * N;
  w += wb * N * (K * BITS / 32);
  scales += wb * N * (K / GS);
  biases += wb * N * (K / GS);

  const int64_t k_begin = (int64_t)ks * k_split;
  const int64_t k_end = min(K, k_begin + k_split);
  const int ntiles = (int)((k_end - k_begin) / 64);
  const int64_t chunk = k_end - k_begin;
  const int64_t row_stride = chunk * 2 + 16;  // bytes per staged x row (+16 breaks bank aliasing)

  // ---- stage x[:, k_begin:k_end] into LDS in operand slot order -----------
  const int64_t blocks8 = chunk / 8;
  for (int64_t i = tid; i < M * blocks8; i += blockDim.x) {
    const int64_t m = i / blocks8, kb = i % blocks8;
    u32x4_t d = *reinterpret_cast<const u32x4_t*>(x + m * K + k_begin + kb * 8);
    *reinterpret_cast<u32x4_t*>(smem + m * row_stride + kb * 16) = permute8<CO::ORDER>(d);
  }
  __syncthreads();

  // ---- this lane's weight row and codes for every tile --------------------
  const int ln = lane & 15;       // column (weight row) within the wave's 16
  const int lg = lane >> 4;       // lane group: k sub-range 16*lg within a tile
  const int64_t n0 = (int64_t)blockIdx.x * QMV_COLS + wave * 16;
  const int64_t n = n0 + ln;
  const int64_t nl = n < N ? n : N - 1;  // clamp loads; stores are masked
  constexpr int WPT = BITS / 2;          // packed words per lane per tile (16 codes)
  const int64_t wrow = K * BITS / 32;
  uint32_t wreg[QMV_MAXT][WPT];
  float sreg[QMV_MAXT], breg[QMV_MAXT];
#pragma unroll
  for (int t = 0; t < QMV_MAXT; t++) {
    if (t < ntiles) {
      const int64_t k = k_begin + t * 64 + lg * 16;
      const uint32_t* src = w + nl * wrow + k * BITS / 32;
      if constexpr (WPT == 2) {
        uint2 v = *reinterpret_cast<const uint2*>(src);
        wreg[t][0] = v.x;
        wreg[t][WPT - 1] = v.y;
      } else {
        uint4 v = *reinterpret_cast<const uint4*>(src);
        wreg[t][0] = v.x;
        wreg[t][1 % WPT] = v.y;
        wreg[t][2 % WPT] = v.z;
        wreg[t][3 % WPT] = v.w;
      }
      const int64_t gi = nl * (K / GS) + (k_begin + t * 64) / GS;
      sreg[t] = Conv<T>::from_bits(scales[gi]);
      breg[t] = Conv<T>::from_bits(biases[gi]);
    }
  }

  const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};
  f32x4_t yacc[MB];
#pragma unroll
  for (int rb = 0; rb < MB; rb++) yacc[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < QMV_MAXT; t++) {
    if (t < ntiles) {
      u32x4_t b0, b1;
      if constexpr (BITS == 4) {
        b0 = CodeOps<T, 4>::operand(wreg[t][0]);
        b1 = CodeOps<T, 4>::operand(wreg[t][WPT - 1]);
      } else {
        b0 = CodeOps<T, BITS>::operand(wreg[t][0], wreg[t][1 % WPT]);
        b1 = CodeOps<T, BITS>::operand(wreg[t][2 % WPT], wreg[t][3 % WPT]);
      }
      const float s = sreg[t];
      const float bb = breg[t] - CO::OFFSET * s;
#pragma unroll
      for (int rb = 0; rb < MB; rb++) {
        int64_t m = rb * 16 + ln;
        m = m < M ? m : M - 1;
        const uint8_t* xr = smem + m * row_stride + (t * 8 + lg * 2) * 16;
        const u32x4_t a0 = *reinterpret_cast<const u32x4_t*>(xr);
        const u32x4_t a1 = *reinterpret_cast<const u32x4_t*>(xr + 16);
        // D = x (rows) . codes (cols): x is the A operand, codes the B operand
        f32x4_t acc = Mma<T>::mma(a0, b0, f32x4_t{0.f, 0.f, 0.f, 0.f});
        acc = Mma<T>::mma(a1, b1, acc);
        f32x4_t xs = Mma<T>::mma(a0, ones, f32x4_t{0.f, 0.f, 0.f, 0.f});
        xs = Mma<T>::mma(a1, ones, xs);
#pragma unroll
        for (int i = 0; i < 4; i++) yacc[rb][i] += s * acc[i] + bb * xs[i];
      }
    }
  }

  // ---- write: D layout row = 4*lg + i, col = ln ---------------------------
  if (nks == 1) {
    if (n < N) {
#pragma unroll
      for (int rb = 0; rb < MB; rb++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int64_t m = rb * 16 + lg * 4 + i;
          if (m < M) y[m * N + n] = (uint16_t)Conv<T>::to_bits(yacc[rb][i]);
        }
    }
    return;
  }
  float* part = partial + (bidx * nks + ks) * M * N;
  if (n < N) {
#pragma unroll
    for (int rb = 0; rb < MB; rb++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int64_t m = rb * 16 + lg * 4 + i;
        if (m < M) part[m * N + n] = yacc[rb][i];
      }
  }
  __threadfence();
  __syncthreads();
  __shared__ uint32_t last;
  if (tid == 0) {
    uint32_t* ctr = counters + bidx * gridDim.x + blockIdx.x;
    last = atomicAdd(ctr, 1u) == (uint32_t)(nks - 1);
    if (last) *ctr = 0;  // leave the counter at zero for the next launch
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  const int64_t ncols = min((int64_t)QMV_COLS, N - (int64_t)blockIdx.x * QMV_COLS);
  for (int64_t i = tid; i < M * ncols; i += blockDim.x) {
    const int64_t m = i / ncols, c = (int64_t)blockIdx.x * QMV_COLS + i % ncols;
    float acc = 0.f;
    for (int k = 0; k < nks; k++) acc += partial[((bidx * nks + k) * M + m) * N + c];
    y[m * N + c] = (uint16_t)Conv<T>::to_bits(acc);
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

template <typename T, int BITS, int GS>
int launch_qmv(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
               const void* biases, int64_t w_rep, int64_t N, void* y, hipStream_t s) {
  const int64_t col_groups = (N + QMV_COLS - 1) / QMV_COLS;
  const int64_t tiles = K / 64;
  // enough k splits for ~8 waves per CU, each split at most QMV_MAXT tiles
  const int64_t want_wgs = (int64_t)mlxq::device_cu_count() * 2;
  int64_t nks = (want_wgs + col_groups * batch - 1) / (col_groups * batch);
  // staged activations stay within 64 KiB of LDS
  int64_t max_tiles = ((65536 / M) - 16) / 128;
  if (max_tiles > QMV_MAXT) max_tiles = QMV_MAXT;
  if (max_tiles < 1) return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: M too large to stage");
  const int64_t min_ks = (tiles + max_tiles - 1) / max_tiles;
  if (nks < min_ks) nks = min_ks;
  if (nks > tiles) nks = tiles;
  if (nks < 1) nks = 1;
  const int64_t tiles_per = (tiles + nks - 1) / nks;
  nks = (tiles + tiles_per - 1) / tiles_per;
  const int64_t k_split = tiles_per * 64;
  const int64_t rows_staged = M;
  const size_t lds = (size_t)rows_staged * (size_t)(k_split * 2 + 16);
  if (lds > 65536) return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: staged activations exceed LDS");
  float* partial = nullptr;
  uint32_t* counters = nullptr;
  if (nks > 1) {
    void* pws = nullptr;
    const size_t pbytes = (size_t)batch * nks * M * N * sizeof(float);
    int rc = mlxq::workspace(pbytes, (size_t)(batch * col_groups), &counters, &pws, s);
    if (rc) return rc;
    partial = reinterpret_cast<float*>(pws);
  }
  dim3 grid((unsigned)col_groups, (unsigned)nks, (unsigned)batch);
  const int mb = (int)((M + 15) / 16);
#define QMV_LAUNCH(MBV)                                                                                     \
  hipLaunchKernelGGL((qmv_mfma_kernel<T, BITS, GS, MBV>), grid, dim3(256), lds, s, (const uint16_t*)x, M, K, w, \
                     (const uint16_t*)scales, (const uint16_t*)biases, N, w_rep, k_split, (uint16_t*)y, partial,  \
                     counters)
  switch (mb) {
    case 1: QMV_LAUNCH(1); break;
    case 2: QMV_LAUNCH(2); break;
    case 3: QMV_LAUNCH(3); break;
    case 4: QMV_LAUNCH(4); break;
    default: return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: M > 64");
  }
#undef QMV_LAUNCH
  MLXQ_LAUNCHED("qmv_mfma_kernel");
  return MLXQ_OK;
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
