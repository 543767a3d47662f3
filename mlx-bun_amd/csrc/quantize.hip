// quantize.hip -- MLX affine quantize / dequantize and the fused
// quantize-on-append into KV caches (gfx950).
//
// Quantize is HBM-bound byte work: each group of `gs` elements is owned by
// gs/8 consecutive lanes, each lane loading 8 elements with one 16-byte load
// (two for fp32), min/max reduced with lane shuffles inside the group, and
// the codes of a lane written as whole words (coalesced across the group).
#include "mlxq_internal.h"

namespace {

template <typename T>
struct Load8;
template <>
struct Load8<BF16> {
  __device__ static void run(const void* base, int64_t elem, float v[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
  }
};
template <>
struct Load8<F16> {
  __device__ static void run(const void* base, int64_t elem, float v[8]) {
    uint4 u = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(base) + elem);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = f16_bits_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = f16_bits_to_f32(w[i] >> 16);
    }
  }
};
template <>
struct Load8<F32> {
  __device__ static void run(const void* base, int64_t elem, float v[8]) {
    const float4* p = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + elem);
    float4 a = p[0], b = p[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

template <typename T>
__device__ __forceinline__ void store_t(void* base, int64_t i, float f) {
  Conv<T>::store(reinterpret_cast<typename T::storage*>(base), i, f);
}

// One launch covers `heads * rows_per_head` input rows of `dim` elements.
// Input row (h, r) -> output row h*capacity + (write_pos + r) mod capacity.
// (rows_per_head = capacity = rows, write_pos = 0 is plain mx.quantize.)
template <typename T, int BITS, int GS>
__global__ void __launch_bounds__(256) quantize_kernel(const void* __restrict__ x, int64_t heads, int64_t rows_per_head,
                                                        int64_t dim, uint32_t* __restrict__ packed,
                                                        void* __restrict__ scales, void* __restrict__ biases,
                                                        int64_t capacity, int64_t write_pos) {
  constexpr int LPG = GS / 8;  // lanes per group
  constexpr float N_BINS = (float)((1 << BITS) - 1);
  const int64_t groups_per_row = dim / GS;
  const int64_t total_groups = heads * rows_per_head * groups_per_row;
  const int64_t words_per_row = dim * BITS / 32;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int li = (int)(tid % LPG);
  int64_t gidx = tid / LPG;
  const bool active = gidx < total_groups;
  if (!active) gidx = 0;  // keep every lane in the shuffles with an in-bounds load

  const int64_t in_row = gidx / groups_per_row;
  const int64_t g = gidx % groups_per_row;
  const int64_t head = in_row / rows_per_head;
  const int64_t r = in_row % rows_per_head;
  const int64_t out_row = head * capacity + (write_pos + r) % capacity;

  float v[8];
  Load8<T>::run(x, in_row * dim + g * GS + li * 8, v);
  float mn = v[0], mx = v[0];
#pragma unroll
  for (int i = 1; i < 8; i++) {
    mn = fminf(mn, v[i]);
    mx = fmaxf(mx, v[i]);
  }
#pragma unroll
  for (int m = 1; m < LPG; m <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, m));
    mx = fmaxf(mx, __shfl_xor(mx, m));
  }
  // MLX affine scheme (ops.quantize, src/mlx/ops.ts:615-641): the group edge
  // with the larger magnitude is represented exactly.
  float scale = fmaxf((mx - mn) / N_BINS, 1e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  scale = side ? scale : -scale;
  const float edge = side ? mn : mx;
  const float q0 = roundf(edge / scale);  // round half away from zero
  float bias = 0.0f;
  if (q0 != 0.0f) {
    scale = edge / q0;
    bias = edge;
  }
  uint32_t code[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float c = roundf((v[i] - bias) / scale);
    c = fminf(fmaxf(c, 0.0f), N_BINS);
    code[i] = (uint32_t)c;
  }
  const int64_t wbase = out_row * words_per_row;
  const int64_t elem0 = g * GS + li * 8;  // element index within the row
  if (BITS == 8) {
    uint32_t w0 = code[0] | (code[1] << 8) | (code[2] << 16) | (code[3] << 24);
    uint32_t w1 = code[4] | (code[5] << 8) | (code[6] << 16) | (code[7] << 24);
    if (active) *reinterpret_cast<uint2*>(packed + wbase + elem0 / 4) = make_uint2(w0, w1);
  } else if (BITS == 4) {
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) w |= code[i] << (4 * i);
    if (active) packed[wbase + elem0 / 8] = w;
  } else {  // BITS == 2: two lanes share one word
    uint32_t h = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) h |= code[i] << (2 * i);
    uint32_t other = __shfl_xor(h, 1);
    if (active && (li & 1) == 0) packed[wbase + elem0 / 16] = h | (other << 16);
  }
  if (active && li == 0) {
    store_t<T>(scales, out_row * groups_per_row + g, scale);
    store_t<T>(biases, out_row * groups_per_row + g, bias);
  }
}

// out = T(fma(scale, code, bias)): one thread per packed word.
template <typename T, int BITS>
__global__ void __launch_bounds__(256) dequantize_kernel(const uint32_t* __restrict__ packed, const void* __restrict__ scales,
                                                          const void* __restrict__ biases, int64_t rows, int64_t dim,
                                                          int gs, const uint32_t* __restrict__ ids, int64_t table_rows,
                                                          void* __restrict__ out) {
  // out row r dequantizes table row ids[r] (r itself without ids); an id
  // outside [0, table_rows) gives a zero row
  constexpr int E = 32 / BITS;
  const int64_t words_per_row = dim / E;
  const int64_t total = rows * words_per_row;
  const int64_t groups_per_row = dim / gs;
  using S = typename T::storage;
  for (int64_t wi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; wi < total;
       wi += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = wi / words_per_row, word = wi % words_per_row;
    const int64_t d0 = word * E;
    S* o = reinterpret_cast<S*>(out) + row * dim + d0;
    int64_t src = row;
    if (ids) {
      src = ids[row];
      if (src >= table_rows) {
#pragma unroll
        for (int i = 0; i < E; i++) Conv<T>::store(o, i, 0.f);
        continue;
      }
    }
    const int64_t gi = src * groups_per_row + d0 / gs;
    const float s = Conv<T>::load(reinterpret_cast<const S*>(scales), gi);
    const float b = Conv<T>::load(reinterpret_cast<const S*>(biases), gi);
    const uint32_t w = packed[src * words_per_row + word];
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float c = (float)((w >> (BITS * i)) & ((1u << BITS) - 1u));
      Conv<T>::store(o, i, __builtin_fmaf(s, c, b));
    }
  }
}

template <typename T, int BITS>
int launch_quantize_gs(const void* x, int64_t heads, int64_t rph, int64_t dim, int gs, uint32_t* packed,
                       void* scales, void* biases, int64_t cap, int64_t pos, hipStream_t s) {
  const int64_t groups = heads * rph * (dim / gs);
  const int64_t threads = groups * (gs / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return mlxq::fail(MLXQ_ERR_ARGUMENT, "quantize: tensor too large");
  switch (gs) {
    case 32:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 32>), dim3((unsigned)blocks), dim3(256), 0, s, x, heads, rph, dim,
                         packed, scales, biases, cap, pos);
      break;
    case 64:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 64>), dim3((unsigned)blocks), dim3(256), 0, s, x, heads, rph, dim,
                         packed, scales, biases, cap, pos);
      break;
    case 128:
      hipLaunchKernelGGL((quantize_kernel<T, BITS, 128>), dim3((unsigned)blocks), dim3(256), 0, s, x, heads, rph, dim,
                         packed, scales, biases, cap, pos);
      break;
    default:
      return mlxq::fail(MLXQ_ERR_ARGUMENT, "group_size must be 32, 64 or 128");
  }
  MLXQ_LAUNCHED("quantize_kernel");
  return MLXQ_OK;
}

int check_quant_args(int dtype, int64_t dim, int gs, int bits) {
  MLXQ_CHECK(mlxq::dtype_supported(dtype), "dtype must be float16, bfloat16 or float32");
  MLXQ_CHECK(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");
  MLXQ_CHECK(gs == 32 || gs == 64 || gs == 128, "group_size must be 32, 64 or 128");
  MLXQ_CHECK(dim > 0 && dim % gs == 0, "last dimension must be a positive multiple of group_size");
  return MLXQ_OK;
}

int quantize_impl(const void* x, int dtype, int64_t heads, int64_t rph, int64_t dim, int gs, int bits,
                  uint32_t* packed, void* scales, void* biases, int64_t cap, int64_t pos, void* stream) {
  MLXQ_REQUIRE_INIT();
  int rc = check_quant_args(dtype, dim, gs, bits);
  if (rc) return rc;
  MLXQ_CHECK(heads >= 0 && rph >= 0, "negative extent");
  if (heads * rph == 0) return MLXQ_OK;
  MLXQ_CHECK(x && packed && scales && biases, "null buffer");
  MLXQ_CHECK((uintptr_t)x % 16 == 0, "input must be 16-byte aligned");
  hipStream_t s = mlxq::resolve_stream(stream);
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2: return launch_quantize_gs<TT, 2>(x, heads, rph, dim, gs, packed, scales, biases, cap, pos, s);
      case 4: return launch_quantize_gs<TT, 4>(x, heads, rph, dim, gs, packed, scales, biases, cap, pos, s);
      default: return launch_quantize_gs<TT, 8>(x, heads, rph, dim, gs, packed, scales, biases, cap, pos, s);
    }
  });
  return MLXQ_OK;
}

}  // namespace

namespace {

int dequantize_impl(const uint32_t* packed, const void* scales, const void* biases, int dtype, int64_t rows,
                    int64_t dim, int group_size, int bits, const uint32_t* ids, int64_t table_rows, void* out,
                    void* stream) {
  int rc = check_quant_args(dtype, dim, group_size, bits);
  if (rc) return rc;
  MLXQ_CHECK(rows >= 0, "negative rows");
  if (rows == 0) return MLXQ_OK;
  MLXQ_CHECK(packed && scales && biases && out, "null buffer");
  hipStream_t s = mlxq::resolve_stream(stream);
  const int64_t words = rows * dim * bits / 32;
  int64_t blocks = (words + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2:
        hipLaunchKernelGGL((dequantize_kernel<TT, 2>), dim3((unsigned)blocks), dim3(256), 0, s, packed, scales, biases,
                           rows, dim, group_size, ids, table_rows, out);
        break;
      case 4:
        hipLaunchKernelGGL((dequantize_kernel<TT, 4>), dim3((unsigned)blocks), dim3(256), 0, s, packed, scales, biases,
                           rows, dim, group_size, ids, table_rows, out);
        break;
      default:
        hipLaunchKernelGGL((dequantize_kernel<TT, 8>), dim3((unsigned)blocks), dim3(256), 0, s, packed, scales, biases,
                           rows, dim, group_size, ids, table_rows, out);
        break;
    }
  });
  MLXQ_LAUNCHED("dequantize_kernel");
  return MLXQ_OK;
}

}  // namespace

extern "C" {

int mlxq_quantize(const void* w, int dtype, int64_t rows, int64_t dim, int group_size, int bits, uint32_t* packed,
                  void* scales, void* biases, void* stream) {
  return quantize_impl(w, dtype, 1, rows, dim, group_size, bits, packed, scales, biases, rows > 0 ? rows : 1, 0,
                       stream);
}

int mlxq_kv_append(const void* x, int dtype, int64_t heads, int64_t rows_per_head, int64_t dim, int group_size,
                   int bits, uint32_t* packed, void* scales, void* biases, int64_t capacity, int64_t write_pos,
                   void* stream) {
  MLXQ_CHECK(capacity > 0, "capacity must be positive");
  MLXQ_CHECK(rows_per_head <= capacity, "more new rows than cache slots");
  MLXQ_CHECK(write_pos >= 0, "negative write position");
  return quantize_impl(x, dtype, heads, rows_per_head, dim, group_size, bits, packed, scales, biases, capacity,
                       write_pos % capacity, stream);
}


int mlxq_dequantize(const uint32_t* packed, const void* scales, const void* biases, int dtype, int64_t rows,
                    int64_t dim, int group_size, int bits, void* out, void* stream) {
  MLXQ_REQUIRE_INIT();
  return dequantize_impl(packed, scales, biases, dtype, rows, dim, group_size, bits, nullptr, rows, out, stream);
}

int mlxq_embedding_gather(const uint32_t* ids, int64_t n, const uint32_t* packed, const void* scales,
                          const void* biases, int dtype, int64_t vocab, int64_t dim, int group_size, int bits,
                          void* out, void* stream) {
  MLXQ_REQUIRE_INIT();
  MLXQ_CHECK(n >= 0 && vocab >= 0, "negative extent");
  if (n == 0) return MLXQ_OK;
  MLXQ_CHECK(ids, "null ids");
  return dequantize_impl(packed, scales, biases, dtype, n, dim, group_size, bits, ids, vocab, out, stream);
}

}  // extern "C"
