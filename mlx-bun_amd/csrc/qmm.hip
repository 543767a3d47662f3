// qmm.hip -- mx.quantized_matmul for MLX affine-quantized weights (gfx950).
//
// qmv path (transpose = true, M small, bits in {4, 8}, group 64/128,
// T = bf16/f16): the weight stream is the roofline.  A weight tile is 16 rows
// x one 64-byte segment of each row (128 codes at 4 bits, 64 at 8); lane
// (n = l%16, q = l/16) holds 16 contiguous bytes of row n, which become the B
// operand of v_mfma_f32_16x16x32 by the mantissa-OR trick (codes stay exact;
// mfma_common.h).  A k-step takes 8 codes from each lane quarter, so when a
// tile holds QG > 1 quantization groups the MFMA rows are indexed by
// (activation row m, group qg): row (m, qg) carries x[m] only in the lane
// quarters of group qg and zeros elsewhere, and every row's dot stays inside
// one group.  Per tile the 16x16 accumulator gets
//     y[m, n] += s[n, g] * D[(m, g), n] + (b[n, g] - off * s[n, g]) * X[(m, g)]
// where X is the same A operand against a ones operand (sum of x over the
// group).  x is staged once per workgroup in LDS, pre-permuted into the code
// slot order, so per-tile waits only ever cover the weight stream (vector
// loads complete in order, LDS reads have their own counter).
// A workgroup owns 16 R weight rows and all of K; its NW waves take TPW
// consecutive tiles each, issue every weight/scale/bias load of those tiles
// up front (raw buffer loads: rows past N and scales past the row read 0
// without a branch) and reduce their partial rows in LDS (fixed order, no
// cross-workgroup traffic).
//
// Everything else (transpose = false, 2-bit, group 32, fp32 activations,
// larger M) takes the dequantize-to-LDS MFMA kernel or the VALU kernel below.
#include <cstdlib>

#include "mfma_common.h"

namespace {

// weight tiles each qmv wave keeps in flight
#ifndef QMV_WIN
#define QMV_WIN 2
#endif

template <typename T, int BITS, int GS, int MB, int R, int TPW, int MR, int XC>
__global__ void __launch_bounds__(512) qmv_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                  const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, int N, int w_rep,
                                                  uint16_t* __restrict__ y) {
  using CO = CodeOps<T, BITS>;
  constexpr int TILE_K = 512 / BITS;                 // codes per 64-byte row segment
  constexpr int KS = TILE_K / 32;                    // MFMA k-steps per tile
  constexpr int QG = TILE_K > GS ? TILE_K / GS : 1;  // quantization groups per tile (1 or 2)
  constexpr int NGW = TPW * TILE_K / GS;             // groups per wave (a multiple of 4)
  constexpr int SCH = 16 * R * NGW / 4;              // 8-byte scale chunks per wave
  constexpr int SPL = (SCH + 63) / 64;               // ... per lane
  constexpr int XPW = TPW * TILE_K;                  // x values per row per wave
  constexpr float OFF = CO::OFFSET;
  static_assert(QG <= 2 && NGW % 4 == 0, "tile / group geometry");
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar offsets need it
  const int ln = lane & 15, lq = lane >> 4;
  const int bidx = blockIdx.y, wb = bidx / w_rep;
  const int n0 = blockIdx.x * 16 * R;
  const int rows = min(16 * R, N - n0);
  const int G = K / GS, KT = K / TILE_K;
  const uint32_t row_bytes = (uint32_t)K * BITS / 8;
  x += (int64_t)bidx * M * K;
  y += (int64_t)bidx * M * N;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, (uint32_t)(M * K * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + ((int64_t)wb * N + n0) * (row_bytes / 4), (uint32_t)rows * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales + ((int64_t)wb * N + n0) * G, (uint32_t)(rows * G * 2));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(biases + ((int64_t)wb * N + n0) * G, (uint32_t)(rows * G * 2));
  // This wave's tiles [t_first, t_first + TPW) (the last wave's tail tiles
  // are clamped duplicates that add nothing) and its private LDS region:
  // x slice [M][XPW] in code-slot order, then (s, b - off s) as float2
  // [NGW][16R].  After all waves' regions: one zero x row [XPW] shared by the
  // workgroup, the A operand of lanes whose group or row is inactive (every
  // wave writes it before reading it, all with zeros).
  const int t_first = wave * TPW;
  const int k_first = t_first * TILE_K, g_first = k_first / GS;
  const int xchunks = M * XPW / 8;
  const size_t wave_lds = (size_t)M * XPW * 2 + (size_t)NGW * 16 * R * 8;
  uint16_t* xl = reinterpret_cast<uint16_t*>(smem + wave * wave_lds);
  float2* sbl = reinterpret_cast<float2*>(smem + wave * wave_lds + (size_t)M * XPW * 2);
  uint16_t* xz = reinterpret_cast<uint16_t*>(smem + nw * wave_lds);

  // ---- 1. x slice and scales/biases of this wave (coalesced), issued before
  // the weight stream: vector loads complete in order, so waiting for these
  // never waits for weights ---------------------------------------------------
  u32x4_t xst[XC];
#pragma unroll
  for (int c = 0; c < XC; c++) {
    const int ci = lane + 64 * c;  // chunk ci: row ci / (XPW/8), 8 values
    const int m = ci / (XPW / 8), kk = k_first + 8 * (ci % (XPW / 8));
    const uint32_t off = (ci < xchunks && kk < K) ? (uint32_t)(m * K + kk) * 2u : 0x80000000u;
    xst[c] = buf_load128(rx, off, 0u);
  }
  uint32_t sst[SPL][2], bst[SPL][2];
#pragma unroll
  for (int c = 0; c < SPL; c++) {
    const int ci = lane + 64 * c;  // chunk ci: row ci % 16R, groups g_first + 4 (ci / 16R) ..
    const int r = ci % (16 * R), g4 = g_first + 4 * (ci / (16 * R));
    const uint32_t off = (ci < SCH && g4 < G) ? (uint32_t)(r * G + g4) * 2u : 0x80000000u;
    const auto sv = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)off, 0, 0);
    const auto bv = __builtin_amdgcn_raw_buffer_load_b64(rb, (int)off, 0, 0);
    sst[c][0] = sv[0];
    sst[c][1] = sv[1];
    bst[c][0] = bv[0];
    bst[c][1] = bv[1];
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. the weight stream: the first QMV_WIN tiles of this wave ----------
  u32x4_t wr[TPW][R];
  // rows past N sit past the descriptor's end and read 0; the tile offset
  // (inside the row) rides in the scalar offset
  uint32_t wlane[R];
#pragma unroll
  for (int ri = 0; ri < R; ri++) wlane[ri] = (uint32_t)(ln + 16 * ri) * row_bytes + 16u * lq;
  auto issue = [&](int t) {
    const uint32_t toff = (uint32_t)min(t_first + t, KT - 1) * 64u;
#pragma unroll
    for (int ri = 0; ri < R; ri++) wr[t][ri] = buf_load128(rw, wlane[ri], toff);
  };
#pragma unroll
  for (int t = 0; t < QMV_WIN && t < TPW; t++) issue(t);
  __builtin_amdgcn_sched_barrier(0);

  // ---- 3. this wave's LDS region (no workgroup barrier) -------------------
#pragma unroll
  for (int c = 0; c < XC; c++) {
    if (64 * c < xchunks) {  // uniform
      const int ci = lane + 64 * c;
      if (ci < xchunks) *reinterpret_cast<u32x4_t*>(xl + ci * 8) = permute8<CO::ORDER>(xst[c]);
    }
  }
  for (int c = lane; c < XPW / 8; c += 64) *reinterpret_cast<u32x4_t*>(xz + 8 * c) = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int c = 0; c < SPL; c++) {
    const int ci = lane + 64 * c;
    if (ci < SCH) {
      const int r = ci % (16 * R), gl = 4 * (ci / (16 * R));
#pragma unroll
      for (int p = 0; p < 2; p++) {
        const float s0 = Conv<T>::from_bits(sst[c][p] & 0xffffu), s1 = Conv<T>::from_bits(sst[c][p] >> 16);
        const float b0 = Conv<T>::from_bits(bst[c][p] & 0xffffu), b1 = Conv<T>::from_bits(bst[c][p] >> 16);
        sbl[(gl + 2 * p) * 16 * R + r] = make_float2(s0, b0 - OFF * s0);
        sbl[(gl + 2 * p + 1) * 16 * R + r] = make_float2(s1, b1 - OFF * s1);
      }
    }
  }
  // (a wave reads back its own LDS writes in order: no barrier needed)

  // A-operand rows: r = ln + 16 rb = (m, qg); lane quarter lq belongs to group
  // lq * QG / 4 of the tile
  const uint16_t* xa[MB];
#pragma unroll
  for (int rb = 0; rb < MB; rb++) {
    const int r = ln + 16 * rb, m = r / QG, qg = r % QG;
    xa[rb] = ((lq * QG / 4 == qg && m < M) ? xl + m * XPW : xz) + lq * (TILE_K / 4);
  }
  const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};
  const uint32_t magic = opaque(Mma<T>::MAGIC);
  f32x4_t yacc[R][MB];
#pragma unroll
  for (int ri = 0; ri < R; ri++)
#pragma unroll
    for (int rb = 0; rb < MB; rb++) yacc[ri][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // ---- 4. tiles: compute tile t, then request tile t + QMV_WIN --------------
  // (a clamped duplicate tail tile reads zero x and zero scales: adds nothing)
#pragma unroll
  for (int t = 0; t < TPW; t++) {
    f32x4_t D[R][MB], X[MB];
#pragma unroll
    for (int rb = 0; rb < MB; rb++) {
      X[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ri = 0; ri < R; ri++) D[ri][rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < KS; j++) {
      u32x4_t bop[R];
#pragma unroll
      for (int ri = 0; ri < R; ri++) {
        const u32x4_t& wv = wr[t][ri];
        if constexpr (BITS == 4)
          bop[ri] = CodeOps<T, 4>::operand(wv[j], magic);
        else
          bop[ri] = CodeOps<T, BITS>::operand(wv[2 * j], wv[2 * j + 1]);
      }
#pragma unroll
      for (int rb = 0; rb < MB; rb++) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xa[rb] + t * TILE_K + 8 * j);
        X[rb] = Mma<T>::mma(a, ones, X[rb]);
#pragma unroll
        for (int ri = 0; ri < R; ri++) D[ri][rb] = Mma<T>::mma(a, bop[ri], D[ri][rb]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (t + QMV_WIN < TPW) issue(t + QMV_WIN);
    __builtin_amdgcn_sched_barrier(0);
    const int gl = t * TILE_K / GS;
#pragma unroll
    for (int ri = 0; ri < R; ri++) {
      float s[QG], bb[QG];
#pragma unroll
      for (int qg = 0; qg < QG; qg++) {
        const float2 sb = sbl[(gl + qg) * 16 * R + ln + 16 * ri];
        s[qg] = sb.x;
        bb[qg] = sb.y;
      }
      // MR < 4: only rows 0 .. MR-1 (lane quarter 0) reach the output
#pragma unroll
      for (int rb = 0; rb < MB; rb++)
#pragma unroll
        for (int i = 0; i < MR; i++)
          yacc[ri][rb][i] = __builtin_fmaf(s[i % QG], D[ri][rb][i], __builtin_fmaf(bb[i % QG], X[rb][i], yacc[ri][rb][i]));
    }
  }

  // ---- 5. reduce the waves (fixed order) and store --------------------------
  __syncthreads();  // every wave is done with its LDS region
  f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);  // [nw][R * MB][64]
#pragma unroll
  for (int ri = 0; ri < R; ri++)
#pragma unroll
    for (int rb = 0; rb < MB; rb++) red[(wave * R * MB + ri * MB + rb) * 64 + lane] = yacc[ri][rb];
  __syncthreads();
  if (wave < R * MB) {
    const int ri = wave / MB, rb = wave % MB;
    f32x4_t acc = red[wave * 64 + lane];
    for (int wv = 1; wv < nw; wv++) {
      const f32x4_t o = red[(wv * R * MB + wave) * 64 + lane];
      acc[0] += o[0];
      acc[1] += o[1];
      acc[2] += o[2];
      acc[3] += o[3];
    }
    const int n = n0 + 16 * ri + ln;
#pragma unroll
    for (int i = 0; i < 4; i += QG) {
      const int m = (16 * rb + 4 * lq + i) / QG;
      float v = 0.f;
#pragma unroll
      for (int q = 0; q < QG; q++) v += acc[i + q];
      if (m < M && n < N) y[(int64_t)m * N + n] = (uint16_t)Conv<T>::to_bits(v);
    }
  }
}

// ---- dequantize-to-LDS MFMA GEMM (transpose = true, larger M) ------------
//
// The large-M path (MLX dequantizes weight tiles into threadgroup memory for
// its qmm as well): per K-step of 64 codes the workgroup's BN weight rows are
// dequantized (fp32 w = s * c + b) into LDS as a pair of T values, hi = T(w)
// and lo = T(w - hi), next to the BM x 64 tile of x; 32x32x16 MFMAs read both
// from LDS and accumulate x * hi + x * lo in fp32.  hi + lo carries w to
// about 2^-16 relative (a single T rounding costs ~1% on a K = 14336 dot
// product, outside the fp32-reference tolerance).
// LDS is double-buffered: the next K-step's codes and x are loaded into
// registers while the current one computes, then dequantized into the other
// buffer; one barrier per K-step.  Rows past M / N read zeros (buffer loads
// past the descriptor's end) and are not stored.
// 8 codes -> 8 dequantized values w = s * c + b as T pairs: hi = T(w),
// lo = T(w - hi)
template <typename T, int BITS>
__device__ __forceinline__ void dequant8(uint32_t w0, uint32_t w1, float s, float b, u32x4_t& hi, u32x4_t& lo) {
  float v[8];
  if constexpr (BITS == 4) {
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = __builtin_fmaf(s, (float)((w0 >> (4 * e)) & 0xfu), b);
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[e] = __builtin_fmaf(s, (float)((w0 >> (8 * e)) & 0xffu), b);
      v[4 + e] = __builtin_fmaf(s, (float)((w1 >> (8 * e)) & 0xffu), b);
    }
  }
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; p++) {
    h[p] = Mma<T>::pack2(v[2 * p], v[2 * p + 1]);
    const float h0 = Conv<T>::from_bits(h[p] & 0xffffu), h1 = Conv<T>::from_bits(h[p] >> 16);
    l[p] = Mma<T>::pack2(v[2 * p] - h0, v[2 * p + 1] - h1);
  }
  hi = u32x4_t{h[0], h[1], h[2], h[3]};
  lo = u32x4_t{l[0], l[1], l[2], l[3]};
}

template <typename T, int BITS, int GS, int BM, int BN>
__global__ void __launch_bounds__(256) qmm_lds_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases, int N, int w_rep,
                                                      uint16_t* __restrict__ y) {
  constexpr int BK = 64, PITCH = BK + 8;            // LDS row pitch in T elements (bank spread)
  constexpr int WM = BM / 2, WN = BN / 2;            // wave tile (2 x 2 waves)
  constexpr int TM = WM / 32, TN = WN / 32;          // 32x32 MFMA tiles per wave
  constexpr int XL = BM * BK / 8 / 256;              // x 16-byte chunks per thread
  constexpr int CW = BK * BITS / 32;                 // code words per weight row per K-step
  constexpr int WCH = BN * CW / 4;                   // weight 16-byte chunks per K-step
  constexpr int WL = (WCH + 255) / 256;              // ... per thread
  static_assert(XL >= 1 && BM * BK / 8 % 256 == 0, "x tile must split evenly over 256 threads");
  __shared__ __align__(16) uint16_t xs[2][BM * PITCH];
  __shared__ __align__(16) uint16_t ws[2][2][BN * PITCH];  // [buffer][hi, lo]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN, bidx = blockIdx.z, wb = bidx / w_rep;
  const int G = K / GS;
  const uint32_t row_bytes = (uint32_t)K * BITS / 8;
  const int mrows = min(BM, M - m0), nrows = min(BN, N - n0);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + ((int64_t)bidx * M + m0) * K, (uint32_t)(mrows * K * 2));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + ((int64_t)wb * N + n0) * (row_bytes / 4), (uint32_t)nrows * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales + ((int64_t)wb * N + n0) * G, (uint32_t)(nrows * G * 2));
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(biases + ((int64_t)wb * N + n0) * G, (uint32_t)(nrows * G * 2));

  // per-thread chunk coordinates: x chunk c -> row c / 8, k 8 (c % 8);
  // weight chunk c -> row c / (CW / 4), words 4 (c % (CW / 4))
  u32x4_t xr[XL], wr[WL];
  uint32_t sr[WL], br[WL];
  auto load = [&](int kt) {
    const uint32_t k0 = (uint32_t)kt * BK;
#pragma unroll
    for (int i = 0; i < XL; i++) {
      const int c = tid + 256 * i;
      xr[i] = buf_load128(rx, ((uint32_t)(c / 8) * (uint32_t)K + k0 + 8u * (c % 8)) * 2u, 0u);
    }
#pragma unroll
    for (int i = 0; i < WL; i++) {
      const int c = tid + 256 * i, r = c / (CW / 4), q = c % (CW / 4);
      const bool ok = WCH % 256 == 0 || c < WCH;
      wr[i] = buf_load128(rw, ok ? (uint32_t)r * row_bytes + k0 * BITS / 8 + 16u * q : 0x80000000u, 0u);
      const uint32_t so = ((uint32_t)r * (uint32_t)G + (k0 + 16u * q * 8u / BITS) / GS) * 2u;
      sr[i] = buf_load16(rs, ok ? so : 0x80000000u, 0u);
      br[i] = buf_load16(rb, ok ? so : 0x80000000u, 0u);
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < XL; i++) {
      const int c = tid + 256 * i;
      *reinterpret_cast<u32x4_t*>(&xs[buf][(c / 8) * PITCH + 8 * (c % 8)]) = xr[i];
    }
#pragma unroll
    for (int i = 0; i < WL; i++) {
      const int c = tid + 256 * i, r = c / (CW / 4), q = c % (CW / 4);
      if (WCH % 256 != 0 && c >= WCH) continue;
      const float sc = Conv<T>::from_bits(sr[i]), bi = Conv<T>::from_bits(br[i]);
      constexpr int VPW = 32 / BITS;  // values per word
      uint16_t* dh = &ws[buf][0][r * PITCH + q * 4 * VPW];
      uint16_t* dl = &ws[buf][1][r * PITCH + q * 4 * VPW];
#pragma unroll
      for (int j = 0; j < (BITS == 4 ? 4 : 2); j++) {
        u32x4_t hv, lv;
        if constexpr (BITS == 4)
          dequant8<T, 4>(wr[i][j], 0u, sc, bi, hv, lv);
        else
          dequant8<T, 8>(wr[i][2 * j], wr[i][2 * j + 1], sc, bi, hv, lv);
        *reinterpret_cast<u32x4_t*>(dh + 8 * j) = hv;
        *reinterpret_cast<u32x4_t*>(dl + 8 * j) = lv;
      }
    }
  };

  f32x16_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

  const int KT = K / BK;
  load(0);
  stash(0);
  __syncthreads();
  const int lr = lane & 31, lk = 8 * (lane >> 5);
  for (int kt = 0; kt < KT; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < KT) load(kt + 1);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ks++) {
      u32x4_t a[TM], bh[TN], bl[TN];
#pragma unroll
      for (int i = 0; i < TM; i++)
        a[i] = *reinterpret_cast<const u32x4_t*>(&xs[buf][(wm * WM + 32 * i + lr) * PITCH + 16 * ks + lk]);
#pragma unroll
      for (int j = 0; j < TN; j++) {
        bh[j] = *reinterpret_cast<const u32x4_t*>(&ws[buf][0][(wn * WN + 32 * j + lr) * PITCH + 16 * ks + lk]);
        bl[j] = *reinterpret_cast<const u32x4_t*>(&ws[buf][1][(wn * WN + 32 * j + lr) * PITCH + 16 * ks + lk]);
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = mma32<T>(a[i], bl[j], mma32<T>(a[i], bh[j], acc[i][j]));
    }
    if (kt + 1 < KT) stash(buf ^ 1);
    __syncthreads();
  }

  // D[32 x 32]: lane holds column lane % 32, rows 8 (v / 4) + 4 (lane / 32) + v % 4
  uint16_t* yb = y + (int64_t)bidx * M * N;
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      const int n = n0 + wn * WN + 32 * j + lr;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int m = m0 + wm * WM + 32 * i + 8 * (v / 4) + 4 * (lane >> 5) + v % 4;
        if (m < M && n < N) yb[(int64_t)m * N + n] = (uint16_t)Conv<T>::to_bits(acc[i][j][v]);
      }
    }
}

template <typename T, int BITS, int GS>
int launch_qmm_lds(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                   const void* biases, int64_t w_rep, int64_t N, void* y, hipStream_t s) {
#define QMM_L(BMV, BNV)                                                                                          \
  {                                                                                                              \
    dim3 grid((unsigned)((N + BNV - 1) / BNV), (unsigned)((M + BMV - 1) / BMV), (unsigned)batch);              \
    hipLaunchKernelGGL((qmm_lds_kernel<T, BITS, GS, BMV, BNV>), grid, dim3(256), 0, s, (const uint16_t*)x, (int)M, \
                       (int)K, w, (const uint16_t*)scales, (const uint16_t*)biases, (int)N, (int)w_rep,          \
                       (uint16_t*)y);                                                                            \
  }
  // big tiles once they still give every CU a workgroup
  if (M >= 128 && ((N + 127) / 128) * ((M + 127) / 128) * batch >= mlxq::device_cu_count())
    QMM_L(128, 128)
  else
    QMM_L(64, 64)
#undef QMM_L
  MLXQ_LAUNCHED("qmm_lds_kernel");
  return MLXQ_OK;
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

// Launch geometry for the qmv kernel, or false when the shape does not fit
// it (then the general kernels run).
struct QmvPlan {
  int R, TPW, NW, MB, MR, XC;  // XC: x chunks (8 values) each lane stages, 8 or 16
  size_t lds;
};

// MLXQ_QMV_TPW (4, 8 or 16) overrides the tiles each wave streams.
int qmv_tpw_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_QMV_TPW");
    return e ? atoi(e) : 0;
  }();
  return v;
}

bool plan_qmv(int bits, int gs, int64_t M, int64_t K, int64_t N, int64_t batch, QmvPlan* p) {
  const int tile_k = 512 / bits;
  const int qg = tile_k > gs ? tile_k / gs : 1;
  const int64_t G = K / gs;
  // scales stage in 8-byte chunks of 4 groups
  if (K % tile_k || K % gs || qg > 2 || G % 4) return false;
  const int64_t rows = M * qg;
  p->MB = rows <= 16 ? 1 : (rows <= 32 ? 2 : 0);
  if (!p->MB) return false;
  p->MR = (p->MB == 1 && rows <= 2) ? 2 : 4;
  const int64_t kt = K / tile_k;
  p->TPW = 0;
  const int ov = qmv_tpw_override();
  for (int tpw : {4, 8, 16}) {
    if ((kt + tpw - 1) / tpw <= 8 && (int64_t)tpw * tile_k / gs % 4 == 0 && (ov == 0 || ov == tpw)) {
      p->TPW = tpw;
      break;
    }
  }
  if (!p->TPW) return false;
  p->NW = (int)((kt + p->TPW - 1) / p->TPW);
  // two row tiles per workgroup when that still gives every CU a workgroup
  p->R = ((N + 31) / 32) * batch >= (int64_t)mlxq::device_cu_count() ? 2 : 1;
  const int64_t xpw = (int64_t)p->TPW * tile_k, ngw = xpw / gs;
  const size_t wave_lds = (size_t)M * xpw * 2 + (size_t)ngw * 16 * p->R * 8;
  const size_t rbytes = (size_t)p->NW * p->R * p->MB * 64 * 16;
  const size_t sbytes = (size_t)p->NW * wave_lds + (size_t)xpw * 2;
  p->lds = sbytes > rbytes ? sbytes : rbytes;
  // x slice staging: 8 or 16 chunks of 8 values per lane
  p->XC = M * xpw <= 8 * 8 * 64 ? 8 : 16;
  return p->lds <= 160 * 1024 && M * xpw <= 16 * 8 * 64;
}

template <typename T, int BITS, int GS, int MB, int R, int TPW, int MR, int XC>
int launch_qmv_inst(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                    const void* biases, int64_t w_rep, int64_t N, void* y, const QmvPlan& p, hipStream_t s) {
  if constexpr (TPW * (512 / BITS) / GS % 4 != 0) {
    return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: tile geometry");
  } else {
    auto kern = qmv_kernel<T, BITS, GS, MB, R, TPW, MR, XC>;
    if (p.lds > 64 * 1024) {
      static bool raised = false;  // per instantiation
      if (!raised) {
        MLXQ_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
        raised = true;
      }
    }
    dim3 grid((unsigned)((N + 16 * R - 1) / (16 * R)), (unsigned)batch);
    hipLaunchKernelGGL(kern, grid, dim3(p.NW * 64), p.lds, s, (const uint16_t*)x, (int)M, (int)K, w,
                       (const uint16_t*)scales, (const uint16_t*)biases, (int)N, (int)w_rep, (uint16_t*)y);
    MLXQ_LAUNCHED("qmv_kernel");
    return MLXQ_OK;
  }
}

template <typename T, int BITS, int GS>
int launch_qmv(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
               const void* biases, int64_t w_rep, int64_t N, void* y, const QmvPlan& p, hipStream_t s) {
#define QMV_I(MBV, RV, TV, MRV, XCV)                                                                            \
  if (p.MB == MBV && p.R == RV && p.TPW == TV && p.MR == MRV && p.XC == XCV)                                    \
    return launch_qmv_inst<T, BITS, GS, MBV, RV, TV, MRV, XCV>(x, batch, M, K, w, scales, biases, w_rep, N, y, p, s);
  QMV_I(1, 1, 4, 2, 8) QMV_I(1, 1, 8, 2, 8) QMV_I(1, 1, 16, 2, 8) QMV_I(1, 2, 4, 2, 8) QMV_I(1, 2, 8, 2, 8)
  QMV_I(1, 2, 16, 2, 8) QMV_I(1, 1, 4, 4, 8) QMV_I(1, 1, 8, 4, 8) QMV_I(1, 1, 16, 4, 8) QMV_I(1, 2, 4, 4, 8)
  QMV_I(1, 2, 8, 4, 8) QMV_I(1, 2, 16, 4, 8) QMV_I(2, 1, 4, 4, 8) QMV_I(2, 1, 8, 4, 8) QMV_I(2, 1, 16, 4, 8)
  QMV_I(2, 2, 4, 4, 8) QMV_I(2, 2, 8, 4, 8) QMV_I(2, 2, 16, 4, 8)
  // larger x slices (e.g. M = 4 at K = 14336, M = 16 at K = 4096)
  QMV_I(1, 1, 16, 4, 16) QMV_I(1, 2, 16, 4, 16) QMV_I(1, 1, 8, 4, 16) QMV_I(1, 2, 8, 4, 16)
  QMV_I(2, 1, 4, 4, 16) QMV_I(2, 2, 4, 4, 16) QMV_I(2, 1, 8, 4, 16) QMV_I(2, 2, 8, 4, 16)
#undef QMV_I
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "qmv: no instance for this plan");
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

  QmvPlan plan;
  const bool qmv_ok = transpose && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                      (group_size == 64 || group_size == 128) && (uintptr_t)x % 16 == 0 &&
                      (uintptr_t)w % 16 == 0 && (uintptr_t)scales % 8 == 0 && (uintptr_t)biases % 8 == 0 &&
                      K * M < ((int64_t)1 << 30) &&
                      plan_qmv(bits, group_size, M, K, N, batch, &plan);
  if (qmv_ok) {
    if (dtype == MLXQ_BFLOAT16) {
      if (bits == 4)
        return group_size == 64 ? launch_qmv<BF16, 4, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s)
                                : launch_qmv<BF16, 4, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s);
      return group_size == 64 ? launch_qmv<BF16, 8, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s)
                              : launch_qmv<BF16, 8, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s);
    }
    if (bits == 4)
      return group_size == 64 ? launch_qmv<F16, 4, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s)
                              : launch_qmv<F16, 4, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s);
    return group_size == 64 ? launch_qmv<F16, 8, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s)
                            : launch_qmv<F16, 8, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, plan, s);
  }

  const bool lds_ok = transpose && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) && K % 64 == 0 &&
                      (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)scales % 2 == 0 &&
                      M * K * 2 < ((int64_t)1 << 31) && N * K < ((int64_t)1 << 31);
  if (lds_ok) {
#define QMM_LDS_T(TT)                                                                                           \
  switch (bits * 1000 + group_size) {                                                                           \
    case 4032: return launch_qmm_lds<TT, 4, 32>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);             \
    case 4064: return launch_qmm_lds<TT, 4, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);             \
    case 4128: return launch_qmm_lds<TT, 4, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);            \
    case 8032: return launch_qmm_lds<TT, 8, 32>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);             \
    case 8064: return launch_qmm_lds<TT, 8, 64>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);             \
    default: return launch_qmm_lds<TT, 8, 128>(x, batch, M, K, w, scales, biases, w_rep, N, y, s);              \
  }
    if (dtype == MLXQ_BFLOAT16) {
      QMM_LDS_T(BF16)
    } else {
      QMM_LDS_T(F16)
    }
#undef QMM_LDS_T
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
