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
// M <= 64 at 4 bits, group 64 (the shapes qmv does not take) runs the
// direct-to-LDS pipelined MFMA GEMM; larger M, other groups and 8-bit take
// the tiled MFMA GEMM; everything else (transpose = false, 2-bit, fp32
// activations) the VALU kernel below.  All of them resolve a batch element
// through a BatchMap, which also serves mx.gather_qmm (an x row map and an
// expert index per element).
#include <algorithm>
#include <cstdlib>

#include "mfma_common.h"

namespace {

// Batch element -> (x batch element, weight matrix).  quantized_matmul:
// xb = b, wb = b / w_rep.  gather_qmm: xb = x_map[b] (or b), wb = w_idx[b].
// An index outside [0, x_batch) / [0, n_w) marks the element's x rows or
// weights as absent: the kernels then read zeros (zero-sized descriptors),
// so the output rows are zeros and no access leaves the arrays.
//
// Work-list mode (seg != null, the tiled GEMM only): seg[0] items, item j =
// (seg[1 + 3j], seg[2 + 3j], seg[3 + 3j]) = (first row, rows, weight index)
// over x / y rows stored one after another (x_batch rows in all) -- the
// sorted rows of mx.gather_qmm, grouped by expert by qmm_segments_kernel.
struct BatchMap {
  const int32_t* x_map;
  const uint32_t* w_idx;
  int64_t x_batch, n_w, w_rep;
  const int32_t* seg = nullptr;
  __device__ __forceinline__ void resolve(int64_t b, int64_t& xb, bool& xok, int64_t& wb, bool& wok) const {
    xb = x_map ? (int64_t)x_map[b] : b;
    wb = w_idx ? (int64_t)w_idx[b] : b / w_rep;
    xok = xb >= 0 && xb < x_batch;
    wok = wb >= 0 && wb < n_w;
    if (!xok) xb = 0;
    if (!wok) wb = 0;
  }
};

// weight tiles each qmv wave keeps in flight: 4 with one MFMA row block
// (M <= 8: a wave's whole stream of 4 tiles is requested with its x slice,
// so the tiles do not queue behind the staging wait), 2 with two (register
// budget)
template <int MB>
constexpr int qmv_window() {
  return MB == 1 ? 4 : 2;
}

template <typename T, int BITS, int GS, int MB, int R, int TPW, int MR, int XC>
__global__ void __launch_bounds__(512) qmv_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                  const uint32_t* __restrict__ w,
                                                  const uint16_t* __restrict__ scales,
                                                  const uint16_t* __restrict__ biases, int N, BatchMap bm,
                                                  int RW, uint16_t* __restrict__ y) {
  using CO = CodeOps<T, BITS>;
  constexpr int TILE_K = 512 / BITS;                 // codes per 64-byte row segment
  constexpr int KS = TILE_K / 32;                    // MFMA k-steps per tile
  constexpr int QG = TILE_K > GS ? TILE_K / GS : 1;  // quantization groups per tile (1 or 2)
  constexpr int NGW = TPW * TILE_K / GS;             // groups per wave (a multiple of 4)
  constexpr int SCH = 16 * R * NGW / 4;              // 8-byte scale chunks per wave
  constexpr int SPL = (SCH + 63) / 64;               // ... per lane
  constexpr int XPW = TPW * TILE_K;                  // x values per row per wave
  constexpr float OFF = CO::OFFSET;
  constexpr int WIN = qmv_window<MB>();
  static_assert(QG <= 2 && NGW % 4 == 0, "tile / group geometry");
  // K need not be a whole number of tiles: the last tile's lanes past K read
  // the next row's codes (or 0 past the matrix) against x slots staged as 0
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar offsets need it
  const int ln = lane & 15, lq = lane >> 4;
  const int bidx = blockIdx.y;
  int64_t xb, wb;
  bool xok, wok;
  bm.resolve(bidx, xb, xok, wb, wok);
  // RW <= 16 R weight rows a workgroup: rows of its last tile past RW read
  // 0 past the descriptors and are not stored
  const int n0 = blockIdx.x * RW;
  const int nrow = min(RW, N - n0);
  const int rows = wok ? nrow : 0;
  const int G = K / GS, KT = (K + TILE_K - 1) / TILE_K;
  const uint32_t row_bytes = (uint32_t)K * BITS / 8;
  x += xb * M * K;
  y += (int64_t)bidx * M * N;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, xok ? (uint32_t)(M * K * 2) : 0u);
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
  if (G % 4 == 0) {  // a row's 4-group chunks are 8-byte aligned
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
  } else {  // the same chunks one group at a time (groups past G read 0)
#pragma unroll
    for (int c = 0; c < SPL; c++) {
      const int ci = lane + 64 * c;
      const int r = ci % (16 * R), g4 = g_first + 4 * (ci / (16 * R));
      uint32_t sv[4], bv[4];
#pragma unroll
      for (int gi = 0; gi < 4; gi++) {
        const uint32_t off = (ci < SCH && g4 + gi < G) ? (uint32_t)(r * G + g4 + gi) * 2u : 0x80000000u;
        sv[gi] = buf_load16(rs, off, 0u);
        bv[gi] = buf_load16(rb, off, 0u);
      }
      sst[c][0] = (sv[0] & 0xffffu) | (sv[1] << 16);
      sst[c][1] = (sv[2] & 0xffffu) | (sv[3] << 16);
      bst[c][0] = (bv[0] & 0xffffu) | (bv[1] << 16);
      bst[c][1] = (bv[2] & 0xffffu) | (bv[3] << 16);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- 2. the weight stream: the first WIN tiles of this wave --------------
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
  for (int t = 0; t < WIN && t < TPW; t++) issue(t);
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

  // ---- 4. tiles: compute tile t, then request tile t + WIN ------------------
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
    if (t + WIN < TPW) issue(t + WIN);
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
  lds_barrier();  // every wave is done with its LDS region
  f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);  // [nw][R * MB][64]
#pragma unroll
  for (int ri = 0; ri < R; ri++)
#pragma unroll
    for (int rb = 0; rb < MB; rb++) red[(wave * R * MB + ri * MB + rb) * 64 + lane] = yacc[ri][rb];
  lds_barrier();
  // output block ob = (ri, rb) is summed and stored by wave ob % nw (a wave
  // takes several blocks when K gave fewer waves than R * MB blocks)
  for (int ob = wave; ob < R * MB; ob += nw) {
    const int ri = ob / MB, rb = ob % MB;
    f32x4_t acc = red[ob * 64 + lane];
    for (int wv = 1; wv < nw; wv++) {
      const f32x4_t o = red[(wv * R * MB + ob) * 64 + lane];
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
      if (m < M && 16 * ri + ln < nrow) y[(int64_t)m * N + n] = (uint16_t)Conv<T>::to_bits(v);
    }
  }
}

// ---- direct-to-LDS pipelined MFMA GEMM for 16 < M <= 64 (4-bit, group 64) --
//
// A workgroup owns 64 weight rows (4 row tiles) and a range of 128-code K
// tiles, for all M activation rows (MB = ceil(M / 16) MFMA row blocks).  One
// K tile per pipeline step.  Its operands reach LDS through direct-to-LDS
// buffer loads (buffer_load_dwordx4 ... lds: each lane's 16 bytes land at
// base + 16 lane), so nothing in flight occupies registers and the rings can
// be deep.  Every load reads 4 rows x 256 contiguous bytes (whole 128-byte
// lines; 16 rows x 64 bytes a load ran the x stream from L2 at a third of
// the rate), its 16-byte pieces XOR-swizzled by row in LDS so that an MFMA
// operand read (16 rows, one piece each) touches every bank once:
//   * weight ring, NSB slots of WB = 4 K tiles (a batch: 64 rows x 256
//     bytes of codes, plus the 64 rows' scales and biases of the 4 tiles,
//     16 bytes a row -- a 4-byte load per row and tile would touch 64 lines
//     for 256 bytes); a code operand (k-step j of tile t, 8 codes of a row)
//     is one 4-byte LDS read per lane;
//   * x ring, NSX slots of one K tile: MB row blocks x 16 rows x 256 bytes;
//     an A operand (8 x values of a row, natural order) is one 16-byte read.
// Waves 0..3 issue the weight loads (row tile w; wave 0 also the scales,
// wave 1 the biases), waves 4..7 the x loads (k-step w - 4 of every row
// block): a wave waits only for its own loads (vector memory counts complete
// in order per wave), so the x stream, which comes from L2, never waits
// behind the weight stream from HBM.  Per step every wave waits for its
// loads of the step, one barrier publishes the step and frees the slots of
// the ones before, and the next loads go out (x: the steps NSX - 2 and
// NSX - 1 ahead; weights, at a batch's first pair: the batch NSB - 1 ahead).
// Every wave computes, two steps at a time: wave w takes group w % 4 of the
// pair (two k-steps) for row tiles 2 (w / 4), 2 (w / 4) + 1 and all MB row
// blocks: X = x against ones and D = x against the exact codes (natural slot
// order: (128 or 1024) + c), folded as acc += s D + (b - OFF s) X.  The four
// group partials of a row tile are summed in LDS in fixed order; K splits
// (blockIdx.z = batch * KS + split) write fp32 partials for
// qmm_splitk_reduce_kernel.  Rows past M or N read zeros (the descriptors
// end there) and are not stored; steps past the split's end load nothing
// (offsets past the descriptors), so every wave issues the same count each
// step and its wait counts stay exact.
template <int MB>
struct DmaShape {
  static constexpr int WB = 4;                   // K tiles per weight batch (256 bytes of a row)
  // weight ring slots (batches) and x ring slots (K tiles); at MB = 4 the
  // x ring gives two slots to the weights (M = 64 on MI355X: 25.4-26.0 ->
  // 24.9 us up, 27.5-27.7 -> 27.2 down; 5 weight batches and 4 x slots, or
  // deeper weight rings at MB = 1, measured the same or slower)
  static constexpr int NSB = MB == 4 ? 4 : MB == 3 ? 3 : MB == 2 ? 4 : 5;
  static constexpr int NSX = MB == 4 ? 4 : 8;
  static constexpr int WSLOT = 16 * 1024;        // codes of a batch: 64 rows x 256 bytes
  static constexpr int SSLOT = 2 * 1024;         // scales, biases of a batch
  static constexpr int XSLOT = MB * 4 * 1024;    // x of a K tile: MB row blocks x 16 rows x 256 bytes
  static constexpr int SOFF = NSB * WSLOT;
  static constexpr int XOFF = SOFF + NSB * SSLOT;
  static constexpr int LDS = XOFF + NSX * XSLOT;
  // The loop runs steps in pairs (c, c + 1), c even; a weight batch is two
  // pairs.  A weight wave issues LB loads per batch: (waves 0, 1) the
  // batch's scales or biases, then its row tile's codes (4 loads of 4 rows x
  // the batch's 256 bytes, so every step needs all of them).  At a batch's
  // first pair it waits for the whole batch: batches up to k + NSB - 2 are
  // out then, NSB - 2 of them after batch k.
  template <int LB>
  static constexpr int wait_w() {
    return (NSB - 2) * LB;
  }
  // x waves: steps up to c + NSX - 3 are out before the pair (two a pair,
  // NSX - 2 in the prologue), NSX - 4 steps follow step c + 1's
  static constexpr int WAIT_X = (NSX - 4) * MB;
  static constexpr int RED = 8 * 2 * MB * 64 * 16;  // per-wave accumulators at the end
  static_assert(LDS <= 160 * 1024 && RED <= LDS, "LDS budget");
  static_assert(WB == 4 && NSB >= 2 && NSX % 2 == 0 && NSX >= 4 && wait_w<5>() <= 63 && WAIT_X <= 63,
                "ring / vmcnt range");
};

// s_barrier that also keeps the compiler from moving memory accesses across
// it.  Unlike a release fence on LDS it does not make the compiler wait for
// the direct-to-LDS loads in flight (those are tracked by vmcnt and waited
// for explicitly before it).
__device__ __forceinline__ void dma_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void dma_load16(__amdgpu_buffer_rsrc_t r, lds_u8* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds, 16, voff, 0, 0, 0);
}
// MFMA B operand from 8 4-bit codes in natural slot order: dword t holds
// (OFF + c_2t, OFF + c_2t+1), OFF + c being exact in T (bf16 128 + c =
// 0x4300 + c, f16 1024 + c = 0x6400 + c: the code is the low byte)
template <typename T>
__device__ __forceinline__ u32x4_t nat_operand(uint32_t w) {
  constexpr uint32_t HI = std::is_same<T, BF16>::value ? 0x43434343u : 0x64646464u;
  const uint32_t lo = w & 0x0f0f0f0fu;         // c0 c2 c4 c6
  const uint32_t hi = (w >> 4) & 0x0f0f0f0fu;  // c1 c3 c5 c7
  const uint32_t p = perm_b32(hi, lo, 0x05010400u);  // c0 c1 c2 c3
  const uint32_t q = perm_b32(hi, lo, 0x07030602u);  // c4 c5 c6 c7
  u32x4_t r;
  r.x = perm_b32(HI, p, 0x04010400u);
  r.y = perm_b32(HI, p, 0x04030402u);
  r.z = perm_b32(HI, q, 0x04010400u);
  r.w = perm_b32(HI, q, 0x04030402u);
  return r;
}

template <typename T, int MB>
__global__ void __launch_bounds__(512) qmm_dma_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                      const uint32_t* __restrict__ w,
                                                      const uint16_t* __restrict__ scales,
                                                      const uint16_t* __restrict__ biases, int N, BatchMap bm, int KS,
                                                      int KTS, uint16_t* __restrict__ y, float* __restrict__ part) {
  using SH = DmaShape<MB>;
  constexpr int NSX = SH::NSX;
  constexpr float OFF = Mma<T>::MAGIC_VAL;
  constexpr uint32_t OOB = 0x80000000u;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lq = lane >> 4;
  const int bidx = blockIdx.z / KS, split = blockIdx.z % KS;
  int64_t xb, wb;
  bool xok, wok;
  bm.resolve(bidx, xb, xok, wb, wok);
  const int n0 = blockIdx.x * 64;
  const int nrows = wok ? min(64, N - n0) : 0;
  const int G = K / 64, KT = K / 128;
  const int sk0 = split * KTS, sk1 = min(KT, sk0 + KTS);
  const int nch = max(sk1 - sk0, 0);
  const uint32_t row_bytes = (uint32_t)K / 2;
  const __amdgpu_buffer_rsrc_t rw =
      make_rsrc(w + ((int64_t)wb * N + n0) * (row_bytes / 4), (uint32_t)nrows * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales + ((int64_t)wb * N + n0) * G, (uint32_t)nrows * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t rb = make_rsrc(biases + ((int64_t)wb * N + n0) * G, (uint32_t)nrows * (uint32_t)G * 2u);
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + xb * M * K, xok ? (uint32_t)M * (uint32_t)K * 2u : 0u);
  lds_u8* const lds = (lds_u8*)smem;  // the same memory through 32-bit LDS addresses
  uint8_t* const xring = smem + SH::XOFF;

  // Batch k = steps WB k .. WB k + WB - 1 covers K tiles tile0(k) .. + WB - 1
  // of the split.  With whole batches only, the workgroups of one XCD
  // (blockIdx.x / 8 consecutive) start at different batches, so they do not
  // all read the same x lines at once.
  constexpr int WB = SH::WB, NSB = SH::NSB;
  const int nb = (nch + WB - 1) / WB;
  const int spread = nch % WB == 0 && nb > 0 ? 1 << (31 - __builtin_clz(nb)) : 1;  // power of 2 <= nb
  const int rot = (int)((blockIdx.x >> 3) + blockIdx.z) & (spread - 1);
  auto tile0 = [&](int k) {  // (past nb: any tile; those loads are masked)
    const int q = k + rot;
    return sk0 + WB * (q >= nb ? q - nb : q);
  };
  // the batch's 16-byte scale / bias load covers tiles sload(k) .. + 3 of
  // every row: the batch's own, shifted back to stay inside the row
  auto sload = [&](int k) { return min(tile0(k), KT - WB); };
  // Loads write each lane's 16 bytes at base + 16 lane, 4 rows x 256 bytes a
  // load (16 lanes a row: whole 128-byte lines; 16 rows x 64 bytes a load
  // reads x from L2 at a third of the rate).  Lane l of a load takes row
  // 4 i + l / 16 of its 16-row block and 16-byte piece (l % 16) ^ (row % 16)
  // of the 256 bytes, so piece P of block row r sits in slot
  // (r / 4) * 64 + (r % 4) * 16 + (P ^ r) (16-byte units): an MFMA operand
  // read (16 rows, one piece each) spreads over all LDS banks.
  auto lane_off = [&](int i, uint32_t pitch) {  // load i of a 16-row block: row 4 i + l / 16
    const int r = 4 * i + (lane >> 4);
    return (uint32_t)r * pitch + (uint32_t)((lane & 15) ^ r) * 16u;
  };
  // waves 0..3: codes of row tile `wave` (loads i < 4)
  uint32_t voff_w[4];
#pragma unroll
  for (int i = 0; i < 4; i++) voff_w[i] = (uint32_t)(16 * wave) * row_bytes + lane_off(i, row_bytes);
  // waves 0, 1: scales / biases (lane: row `lane`, 4 tiles' 8 groups)
  const uint32_t voff_sb = (uint32_t)lane * (uint32_t)G * 2u;
  // waves 4..7: load wave - 4 of every row block
  const uint32_t voff_x = lane_off(wave & 3, (uint32_t)K * 2u);
  auto issue_w = [&](int k) {  // batch k, weight waves: scales / biases first, then the codes
    const int t0 = tile0(k);
    const bool live = WB * k < nch;
    if (wave < 2)
      dma_load16(wave == 0 ? rs : rb, lds + SH::SOFF + (k % NSB) * SH::SSLOT + wave * 1024,
                 live ? voff_sb + (uint32_t)sload(k) * 4u : OOB);
    // past the split's end (a partial batch) the loads read on into the row,
    // or read 0 past the matrix: those tiles are never computed
#pragma unroll
    for (int i = 0; i < 4; i++)
      dma_load16(rw, lds + (k % NSB) * SH::WSLOT + wave * 4096 + i * 1024,
                 live ? voff_w[i] + (uint32_t)t0 * 64u : OOB);
  };
  auto issue_x = [&](int c) {  // step c, x waves
    const int kt = tile0(c / WB) + c % WB;
    lds_u8* slot = lds + SH::XOFF + (c % NSX) * SH::XSLOT + (wave - 4) * 1024;
#pragma unroll
    for (int b = 0; b < MB; b++)
      dma_load16(rx, slot + b * 4096,
                 c < nch ? voff_x + (uint32_t)(16 * b) * (uint32_t)K * 2u + (uint32_t)kt * 256u : OOB);
  };
  auto wait_w = [&]() {
    if (wave < 2)
      wait_vmcnt<SH::template wait_w<5>()>();
    else
      wait_vmcnt<SH::template wait_w<4>()>();
  };
  // 16-byte unit of piece P of row r of a 16-row block
  auto slot16 = [](int r, int P) { return (r >> 2) * 64 + (r & 3) * 16 + (P ^ r); };

  // compute: of each pair of steps, wave w takes group gi = w % 4 (step
  // c + gi / 2, group gi % 2 of its tile) for row tiles 2 h, 2 h + 1
  // (h = w / 4) and every row block: each x operand read serves two row
  // tiles, each row sum X two D tiles
  const int gi = wave & 3, h = wave >> 2;
  f32x4_t acc[2][MB];
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int b = 0; b < MB; b++) acc[r][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};

  if (wave < 4)
    for (int k = 0; k < NSB - 1; k++) issue_w(k);
  else
    for (int c = 0; c < NSX - 2; c++) issue_x(c);
  for (int c = 0; c < nch; c += 2) {
    const int k = c / WB;
    const bool second = (c % WB) != 0;
    if (wave >= 4)
      wait_vmcnt<SH::WAIT_X>();
    else if (!second)
      wait_w();
    dma_barrier();  // steps c, c + 1 in LDS everywhere; the slots of the steps before free
    if (wave >= 4) {
      issue_x(c + NSX - 2);
      issue_x(c + NSX - 1);
    } else if (!second) {
      issue_w(k + NSB - 1);
    }
    const int st = c + (gi >> 1), kg = gi & 1;
    if (st >= nch) continue;  // the odd last step (wave-uniform)
    const uint8_t* ws = smem + (k % NSB) * SH::WSLOT;
    const uint8_t* xs = xring + (st % NSX) * SH::XSLOT;
    const int tb = st % WB;  // the step's tile in the batch
    // (s, b) of group 2 kt + kg of row 16 rt + ln: halfword 2 (kt - sload) + kg
    // of the row's 16 bytes
    float sc[2], bp[2];
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const uint8_t* ss = smem + SH::SOFF + (k % NSB) * SH::SSLOT + (16 * (2 * h + r) + ln) * 16 +
                          (2 * (tile0(k) + st % WB - sload(k)) + kg) * 2;
      sc[r] = Conv<T>::from_bits(*reinterpret_cast<const uint16_t*>(ss));
      bp[r] = Conv<T>::from_bits(*reinterpret_cast<const uint16_t*>(ss + 1024)) - OFF * sc[r];
    }
    // the group's first k-step starts X and D from an inline 0 (no zeroing moves)
    const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
    f32x4_t X[MB], D[2][MB];
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
      const int j = 2 * kg + jj;
      u32x4_t bop[2];
#pragma unroll
      for (int r = 0; r < 2; r++)
        bop[r] = nat_operand<T>(
            *reinterpret_cast<const uint32_t*>(ws + (2 * h + r) * 4096 + slot16(ln, 4 * tb + j) * 16 + 4 * lq));
#pragma unroll
      for (int b = 0; b < MB; b++) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(xs + b * 4096 + slot16(ln, 4 * j + lq) * 16);
        X[b] = Mma<T>::mma(a, ones, jj ? X[b] : zero);
        D[0][b] = Mma<T>::mma(a, bop[0], jj ? D[0][b] : zero);
        D[1][b] = Mma<T>::mma(a, bop[1], jj ? D[1][b] : zero);
      }
    }
#pragma unroll
    for (int r = 0; r < 2; r++)
#pragma unroll
      for (int b = 0; b < MB; b++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          acc[r][b][i] = __builtin_fmaf(sc[r], D[r][b][i], __builtin_fmaf(bp[r], X[b][i], acc[r][b][i]));
  }
  // drain the loads past the end (they land in ring slots) before the LDS is reused
  wait_vmcnt<0>();
  lds_barrier();
  f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);  // [wave][2][MB][64]
#pragma unroll
  for (int r = 0; r < 2; r++)
#pragma unroll
    for (int b = 0; b < MB; b++) red[((wave * 2 + r) * MB + b) * 64 + lane] = acc[r][b];
  lds_barrier();
  // output block (row tile t, row block b): the four group waves of pair
  // t / 2 (waves 4 (t / 2) + g), summed in order g = 0..3
  for (int ob = wave; ob < 4 * MB; ob += 8) {
    const int t = ob / MB, b = ob % MB;
    f32x4_t v = red[(((4 * (t >> 1)) * 2 + (t & 1)) * MB + b) * 64 + lane];
#pragma unroll
    for (int g = 1; g < 4; g++) {
      const f32x4_t o = red[(((4 * (t >> 1) + g) * 2 + (t & 1)) * MB + b) * 64 + lane];
      v[0] += o[0];
      v[1] += o[1];
      v[2] += o[2];
      v[3] += o[3];
    }
    const int n = n0 + 16 * t + ln;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 16 * b + 4 * lq + i;
      if (m < M && n < N) {
        if (KS == 1)
          y[((int64_t)bidx * M + m) * N + n] = (uint16_t)Conv<T>::to_bits(v[i]);
        else
          part[(((int64_t)split * (gridDim.z / KS) + bidx) * M + m) * N + n] = v[i];
      }
    }
  }
}

// ---- tiled MFMA GEMM over exact code operands (transpose = true) ---------
//
// The larger-M path (MLX's qmm stages weight tiles in threadgroup memory as
// well).  A workgroup owns a BM x BN tile of y and a range of K.  Per K-step
// of 64 codes it stages in LDS:
//   * the x tile as T, each 8-value run permuted into the code slot order;
//   * the weight codes as exact MFMA operands OFF + c (CodeOps);
//   * per part of a quant group inside the step (64 values, or 32 for
//     group_size 32): every weight row's (s, b - OFF s).
// The 32x32x16 MFMAs contract one group part at a time into D (x against the
// codes) and X (x against ones: the row sums of x, already in D's layout),
// and the part folds into the fp32 accumulators as acc += s D + (b - OFF s) X:
// the products are exact and only fp32 accumulation rounds, so no rounding of
// dequantized weights to T enters the result.
// Register prefetch runs PF K-steps ahead of the LDS double buffer (one
// barrier per step).  Workgroups of a split K (blockIdx.z = batch * KS +
// split) write fp32 partials that qmm_splitk_reduce_kernel sums in fixed
// split order.  Rows past M / N read zeros and are not stored.
template <int BM, int BN>
struct TileShape {
  static constexpr int WGM = BM >= 64 ? 2 : 1;  // wave grid (4 waves)
  static constexpr int WGN = 4 / WGM;
  static constexpr int WM = BM / WGM, WN = BN / WGN;
  static constexpr int TM = WM / 32, TN = WN / 32;  // 32x32 MFMA tiles per wave
  static constexpr int PF = BM * BN >= 128 * 128 ? 2 : 4;
  static_assert(TM >= 1 && TN >= 1 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
};

template <typename T, int BITS, int GS, int BM, int BN, bool SEG = false>
__global__ void __launch_bounds__(256) qmm_tile_kernel(const uint16_t* __restrict__ x, int M, int K,
                                                       const uint32_t* __restrict__ w,
                                                       const uint16_t* __restrict__ scales,
                                                       const uint16_t* __restrict__ biases, int N, BatchMap bm,
                                                       int KS, int KTS, uint32_t sb_bytes,
                                                       uint16_t* __restrict__ y, float* __restrict__ part) {
  using SH = TileShape<BM, BN>;
  using CO = CodeOps<T, BITS>;
  constexpr int WM = SH::WM, WN = SH::WN, TM = SH::TM, TN = SH::TN, PF = SH::PF;
  constexpr int BK = 64, PITCH = BK + 8;            // LDS row pitch in 16-bit elements (bank spread)
  constexpr int EG = GS < BK ? GS : BK;             // K values per group part
  constexpr int NGK = BK / EG;                      // group parts per K-step
  constexpr int SPG = EG / 16;                      // MFMA k-steps per group part
  constexpr int XL = BM / 32;                       // x 16-byte chunks per thread per K-step
  constexpr int CWR = BK * BITS / 32;               // code words per weight row per K-step
  constexpr int WPT = BN * BITS / 128;              // code words per thread per K-step
  constexpr int UW = BITS / 4;                      // code words per 8-code unit
  constexpr int UPT = WPT / UW;                     // 8-code units per thread
  constexpr float OFF = CO::OFFSET;
  static_assert(CWR % WPT == 0, "a thread's code words stay in one row");
  static_assert(BN * NGK <= 256, "one (s, b) item per thread");

  __shared__ __align__(16) uint16_t xs[2][BM * PITCH];
  __shared__ __align__(16) uint16_t wc[2][BN * PITCH];
  __shared__ __align__(16) float2 sbl[2][NGK][BN];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / SH::WGN, wn = wave % SH::WGN;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  // One item (z = blockIdx.z), or with a work list (SEG, KS = 1) items z,
  // z + gridDim.z, ...: every row block of the list is computed whatever the
  // grid, also for a list longer than it.
  const int z_end = SEG ? bm.seg[0] : (int)blockIdx.z + 1;
  for (int z = blockIdx.z; z < z_end; z += SEG ? (int)gridDim.z : 1) {
    const int bidx = z / KS, split = z % KS;
    int64_t xb = 0, wb, xrow0, yrow0;
    bool xok, wok;
    int Mi = M;
    if constexpr (SEG) {
      const int32_t* it = bm.seg + 1 + 3 * (int64_t)z;
      xrow0 = it[0];
      Mi = it[1];
      wb = it[2];
      xok = xrow0 >= 0 && Mi >= 1 && Mi <= BM && xrow0 + Mi <= bm.x_batch;
      wok = wb >= 0 && wb < bm.n_w;
      if (!xok) xrow0 = 0, Mi = 0;  // nothing read, nothing stored
      if (!wok) wb = 0;
      yrow0 = xrow0;
    } else {
      bm.resolve(bidx, xb, xok, wb, wok);
      xrow0 = xb * M;
      yrow0 = 0;  // stores index (bidx, m) directly
    }
    const int G = K / GS, KT = K / BK;
    const int kb = split * KTS, ke = min(KT, kb + KTS);
    const uint32_t row_bytes = (uint32_t)K * BITS / 8;
    const int mrows = xok ? min(BM, Mi - m0) : 0, nrows = wok ? min(BN, N - n0) : 0;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (xrow0 + m0) * K, (uint32_t)(mrows * K * 2));
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(w + ((int64_t)wb * N + n0) * (row_bytes / 4), (uint32_t)nrows * row_bytes);
    // scales / biases: whole arrays (4-byte aligned), read as the dword that
    // holds the wanted 16-bit value (a 16-bit load feeding the prefetch ring
    // would be widened, and so waited for, right at the load)
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(scales, wok ? sb_bytes : 0u);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(biases, wok ? sb_bytes : 0u);
    const int64_t sb_elem0 = ((int64_t)wb * N + n0) * G;  // tile's first (row, group) element
    constexpr uint32_t OOB = 0x80000000u;  // past every descriptor: reads 0

    // thread -> staging items.  x: chunk c = tid + 256 i -> row c / 8, unit
    // c % 8 (8 values); the 8 units of a row sit in 8 adjacent lanes.
    // codes: words [q, q + WPT) of row wr_row.  (s, b): row sb_row, part sb_e.
    const int wr_row = tid * WPT / CWR, wr_q = tid * WPT % CWR;
    const int sb_row = tid / NGK, sb_e = tid % NGK;
    const bool sb_act = tid < BN * NGK;

    u32x4_t xr[PF][XL];
    uint32_t wr[PF][WPT];
    uint32_t sr[PF], br[PF];
    // element index of (row sb_row, group of part sb_e) in K-step kt
    auto sb_elem = [&](int kt) -> int64_t {
      return sb_elem0 + (int64_t)sb_row * G + ((int64_t)kt * BK + sb_e * EG) / GS;
    };
    // Steps past the split's end re-read its last step (never staged): a
    // masked offset would be a uniform select, which the compiler turns into
    // branches whose loads wait for the whole prefetch ring.
    auto load = [&](int kt, u32x4_t (&xv)[XL], uint32_t (&wv)[WPT], uint32_t& sv, uint32_t& bv) {
      kt = min(kt, ke - 1);
      const uint32_t k0 = (uint32_t)kt * BK;
  #pragma unroll
      for (int i = 0; i < XL; i++) {
        const int c = tid + 256 * i;
        xv[i] = buf_load128(rx, ((uint32_t)(c / 8) * (uint32_t)K + 8u * (c % 8)) * 2u, k0 * 2u);
      }
      const uint32_t wo = (uint32_t)wr_row * row_bytes + 4u * wr_q;
      if constexpr (WPT == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rw, (int)wo, (int)(k0 * BITS / 8), 0);
        wv[0] = v[0];
        wv[1] = v[1];
      } else {
  #pragma unroll
        for (int h = 0; h < WPT / 4; h++) {
          const u32x4_t v = buf_load128(rw, wo + 16u * h, k0 * BITS / 8);
          wv[4 * h] = v.x;
          wv[4 * h + 1] = v.y;
          wv[4 * h + 2] = v.z;
          wv[4 * h + 3] = v.w;
        }
      }
      const uint32_t so = sb_act ? (uint32_t)(2 * sb_elem(kt)) & ~3u : OOB;
      sv = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)so, 0, 0);
      bv = __builtin_amdgcn_raw_buffer_load_b32(rb, (int)so, 0, 0);
    };
    auto stash = [&](const u32x4_t (&xv)[XL], const uint32_t (&wv)[WPT], uint32_t sv, uint32_t bv, int kt,
                     int buf) {
  #pragma unroll
      for (int i = 0; i < XL; i++) {
        const int c = tid + 256 * i, row = c / 8, unit = c % 8;
        *reinterpret_cast<u32x4_t*>(&xs[buf][row * PITCH + 8 * unit]) = permute8<CO::ORDER>(xv[i]);
      }
      const uint32_t magic = opaque(Mma<T>::MAGIC);
  #pragma unroll
      for (int u = 0; u < UPT; u++) {
        u32x4_t op;
        if constexpr (BITS == 4)
          op = CodeOps<T, 4>::operand(wv[u], magic);
        else
          op = CodeOps<T, BITS>::operand(wv[2 * u], wv[2 * u + 1]);
        *reinterpret_cast<u32x4_t*>(&wc[buf][wr_row * PITCH + 8 * (wr_q / UW + u)]) = op;
      }
      if (sb_act) {
        const int sh = 16 * (int)(sb_elem(kt) & 1);
        const float sc = Conv<T>::from_bits((sv >> sh) & 0xffffu), bi = Conv<T>::from_bits((bv >> sh) & 0xffffu);
        sbl[buf][sb_e][sb_row] = make_float2(sc, bi - OFF * sc);
      }
    };

    f32x16_t acc[TM][TN];
  #pragma unroll
    for (int i = 0; i < TM; i++)
  #pragma unroll
      for (int j = 0; j < TN; j++)
  #pragma unroll
        for (int e = 0; e < 16; e++) acc[i][j][e] = 0.f;

    const int lr = lane & 31, lh = lane >> 5;
    const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};
    // A group part's fold is deferred until the next part's MFMAs are issued
    // (where registers allow), so its VALU work overlaps the matrix core; the
    // pending part starts as zeros (folding it adds nothing).
    constexpr bool DEFER = TM * TN <= 2;
    f32x16_t pd[DEFER ? TM : 1][DEFER ? TN : 1], px[DEFER ? TM : 1];
    float2 psb[DEFER ? TN : 1];
  #pragma unroll
    for (int i = 0; i < (DEFER ? TM : 1); i++) {
  #pragma unroll
      for (int v = 0; v < 16; v++) px[i][v] = 0.f;
  #pragma unroll
      for (int j = 0; j < (DEFER ? TN : 1); j++)
  #pragma unroll
        for (int v = 0; v < 16; v++) pd[i][j][v] = 0.f;
    }
  #pragma unroll
    for (int j = 0; j < (DEFER ? TN : 1); j++) psb[j] = make_float2(0.f, 0.f);
    auto fold = [&](const f32x16_t (&d)[TM][TN], const f32x16_t (&xsm)[TM], const float2 (&sb)[TN]) {
  #pragma unroll
      for (int i = 0; i < TM; i++)
  #pragma unroll
        for (int j = 0; j < TN; j++)
  #pragma unroll
          for (int v = 0; v < 16; v++)
            acc[i][j][v] = __builtin_fmaf(sb[j].x, d[i][j][v], __builtin_fmaf(sb[j].y, xsm[i][v], acc[i][j][v]));
    };
    auto compute = [&](int buf) {
  #pragma unroll
      for (int e = 0; e < NGK; e++) {
        f32x16_t d[TM][TN], xsm[TM];
  #pragma unroll
        for (int ss = 0; ss < SPG; ss++) {
          const int kk = 16 * (e * SPG + ss) + 8 * lh;
          u32x4_t a[TM], b[TN];
  #pragma unroll
          for (int i = 0; i < TM; i++)
            a[i] = *reinterpret_cast<const u32x4_t*>(&xs[buf][(wm * WM + 32 * i + lr) * PITCH + kk]);
  #pragma unroll
          for (int j = 0; j < TN; j++)
            b[j] = *reinterpret_cast<const u32x4_t*>(&wc[buf][(wn * WN + 32 * j + lr) * PITCH + kk]);
          f32x16_t z;
  #pragma unroll
          for (int v = 0; v < 16; v++) z[v] = 0.f;
  #pragma unroll
          for (int i = 0; i < TM; i++) {
            xsm[i] = mma32<T>(a[i], ones, ss == 0 ? z : xsm[i]);
  #pragma unroll
            for (int j = 0; j < TN; j++) d[i][j] = mma32<T>(a[i], b[j], ss == 0 ? z : d[i][j]);
          }
        }
        // fold: lane column n = wn WN + 32 j + lr, rows 8 (v/4) + 4 lh + v%4
        float2 sb[TN];
  #pragma unroll
        for (int j = 0; j < TN; j++) sb[j] = sbl[buf][e][wn * WN + 32 * j + lr];
        if constexpr (DEFER) {
          fold(pd, px, psb);
  #pragma unroll
          for (int i = 0; i < TM; i++) {
            px[i] = xsm[i];
  #pragma unroll
            for (int j = 0; j < TN; j++) pd[i][j] = d[i][j];
          }
  #pragma unroll
          for (int j = 0; j < TN; j++) psb[j] = sb[j];
        } else {
          fold(d, xsm, sb);
        }
      }
    };

  #pragma unroll
    for (int p = 0; p < PF; p++) load(kb + p, xr[p], wr[p], sr[p], br[p]);
    stash(xr[0], wr[0], sr[0], br[0], kb, 0);
    lds_barrier();
    // Loads are unconditional (steps past the end re-read the last one) so the
    // count of loads between any two points is static and the waits before a
    // stash leave the later slots in flight.
    for (int k0 = kb; k0 < ke; k0 += PF) {
  #pragma unroll
      for (int j = 0; j < PF; j++) {
        const int kt = k0 + j;
        load(kt + PF, xr[j], wr[j], sr[j], br[j]);  // slot j was staged for step kt
        if (kt < ke) {  // workgroup-uniform
          const int buf = (kt - kb) & 1;
          compute(buf);
          if (kt + 1 < ke)
            stash(xr[(j + 1) % PF], wr[(j + 1) % PF], sr[(j + 1) % PF], br[(j + 1) % PF], kt + 1, buf ^ 1);
          lds_barrier();
        }
      }
    }

    if constexpr (DEFER) fold(pd, px, psb);

    // D[32 x 32]: lane holds column lane % 32, rows 8 (v / 4) + 4 (lane / 32) + v % 4
  #pragma unroll
    for (int i = 0; i < TM; i++)
  #pragma unroll
      for (int j = 0; j < TN; j++) {
        const int n = n0 + wn * WN + 32 * j + lr;
  #pragma unroll
        for (int v = 0; v < 16; v++) {
          const int m = m0 + wm * WM + 32 * i + 8 * (v / 4) + 4 * lh + v % 4;
          if (m < Mi && n < N) {
            if constexpr (SEG)
              y[(yrow0 + m) * N + n] = (uint16_t)Conv<T>::to_bits(acc[i][j][v]);
            else if (KS == 1)
              y[((int64_t)bidx * M + m) * N + n] = (uint16_t)Conv<T>::to_bits(acc[i][j][v]);
            else
              part[(((int64_t)split * gridDim.z / KS + bidx) * M + m) * N + n] = acc[i][j][v];
          }
        }
      }
  }  // work items
}

// Work list of mx.gather_qmm over sorted rows: rows with equal consecutive
// indices form one expert's run, cut into blocks of at most BM rows; item j
// = (first row, rows, expert) at seg[1 + 3j], the count at seg[0] (at most R
// items).  One workgroup takes the rows 4096 at a time, 4 consecutive rows a
// thread, all of a pass's index loads in flight at once: a max-scan of run
// starts gives each row its run's start, a sum-scan numbers the block starts
// (within the thread, then lane shuffles, then the 16 wave totals).  The
// pass's item starts stay in LDS, so every item's length (the distance to
// the next start) is written without reading global memory back; the last
// item of a pass is closed by the next pass's first start (or R).  Every run
// start is a block start, so the items tile the rows in order; unsorted
// indices only give shorter runs.
__global__ void __launch_bounds__(1024) qmm_segments_kernel(const uint32_t* __restrict__ idx, int R, int BM,
                                                            int32_t* seg) {
  constexpr int RPT = 4, PASS = 1024 * RPT;
  __shared__ int istart[PASS];  // this pass's item starts, in order
  __shared__ int wmax[16], wsum[16];
  __shared__ int carry_start, carry_count, last_start, pass_items;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (tid == 0) carry_start = 0, carry_count = 0, last_start = 0;
  __syncthreads();
  for (int base = 0; base < R; base += PASS) {
    const int r0 = base + RPT * tid;
    uint32_t v[RPT];
#pragma unroll
    for (int k = 0; k < RPT; k++) v[k] = r0 + k < R ? idx[r0 + k] : 0u;
    const uint32_t before = r0 > 0 && r0 <= R ? idx[r0 - 1] : 0u;
    // latest run start at or before each of this thread's rows (-1: none yet)
    int ls[RPT], cur = -1;
#pragma unroll
    for (int k = 0; k < RPT; k++) {
      const int r = r0 + k;
      if (r < R && (r == 0 || (k ? v[k - 1] : before) != v[k])) cur = r;
      ls[k] = cur;
    }
    int m = cur;  // inclusive max-scan over the threads
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(m, off);
      if (lane >= off) m = max(m, o);
    }
    if (lane == 63) wmax[wave] = m;
    __syncthreads();
    int prior = carry_start;  // run start carried into this thread's first row
    for (int w = 0; w < wave; w++) prior = max(prior, wmax[w]);
    const int up = __shfl_up(m, 1);
    if (lane > 0) prior = max(prior, up);
    int nf = 0;
    bool f[RPT];
#pragma unroll
    for (int k = 0; k < RPT; k++) {
      const int r = r0 + k;
      const int rs = ls[k] >= 0 ? ls[k] : prior;
      f[k] = r < R && (r - rs) % BM == 0;  // a block starts here
      nf += f[k] ? 1 : 0;
    }
    int c = nf;  // inclusive sum-scan of block starts over the threads
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_up(c, off);
      if (lane >= off) c += o;
    }
    if (lane == 63) wsum[wave] = c;
    __syncthreads();
    for (int w = 0; w < wave; w++) c += wsum[w];
    int pos = c - nf;  // this thread's first item in the pass
    const int cc = carry_count;
#pragma unroll
    for (int k = 0; k < RPT; k++) {
      if (f[k]) {
        istart[pos] = r0 + k;
        seg[1 + 3 * (cc + pos)] = r0 + k;
        seg[3 + 3 * (cc + pos)] = (int32_t)v[k];
        pos++;
      }
    }
    if (tid == 1023) {
      pass_items = c;
      int mx = carry_start;
      for (int w = 0; w < 16; w++) mx = max(mx, wmax[w]);
      carry_start = mx;  // read by no thread before the barrier below
    }
    __syncthreads();
    const int total = pass_items;
    for (int jj = tid; jj + 1 < total; jj += 1024) seg[2 + 3 * (cc + jj)] = istart[jj + 1] - istart[jj];
    if (tid == 0 && total > 0) {
      if (cc > 0) seg[2 + 3 * (cc - 1)] = istart[0] - last_start;  // the previous pass's last item
      last_start = istart[total - 1];
      carry_count = cc + total;
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (carry_count > 0) seg[2 + 3 * (carry_count - 1)] = R - last_start;
    seg[0] = carry_count;
  }
}

// y = T(sum over splits of the fp32 partials), fixed split order.
template <typename T>
__global__ void __launch_bounds__(256) qmm_splitk_reduce_kernel(const float4* __restrict__ part, int64_t n4, int KS,
                                                                uint2* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  float4 a = part[i];
  for (int k0 = 1; k0 < KS; k0 += 8) {
    float4 b[8];
#pragma unroll
    for (int k = 0; k < 8; k++) b[k] = k0 + k < KS ? part[(int64_t)(k0 + k) * n4 + i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int k = 0; k < 8; k++) {
      a.x += b[k].x;
      a.y += b[k].y;
      a.z += b[k].z;
      a.w += b[k].w;
    }
  }
  y[i] = make_uint2(Conv<T>::to_bits(a.x) | (Conv<T>::to_bits(a.y) << 16),
                    Conv<T>::to_bits(a.z) | (Conv<T>::to_bits(a.w) << 16));
}

// Tile and split choice: 32 x 128 for M <= 32 and 64 x 128 for M <= 64
// (x staging amortised over 128 weight rows), 128 x 128 once those give every
// CU a workgroup, else 64 x 64; K is split (fp32 partials + reduce) until every CU
// has a workgroup, keeping at least 8 K-steps per split.
// MLXQ_QMM_KS: fixed K split (power of two) for the tiled and direct-to-LDS GEMMs (tuning)
int qmm_ks_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_QMM_KS");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <typename T, int BITS, int GS, int BM, int BN>
int launch_qmm_tile_inst(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                         const void* biases, const BatchMap& bm, int64_t N, void* y, hipStream_t s) {
  const int64_t tiles = ((N + BN - 1) / BN) * ((M + BM - 1) / BM) * batch;
  const int64_t KT = K / 64;
  const int64_t target = mlxq::device_cu_count();
  int KS = 1;
  const bool can_split = N % 4 == 0 && (uintptr_t)y % 8 == 0;
  // smallest split that gives every CU a workgroup (more only adds fp32
  // partial traffic and contention)
  while (can_split && KS < 64 && tiles * KS < target && KT / (KS * 2) >= 8) KS *= 2;
  const int ov = qmm_ks_override();
  if (ov >= 1 && ov <= 64 && (ov == 1 || can_split)) KS = ov;
  const size_t pbytes = KS > 1 ? (size_t)KS * batch * M * N * sizeof(float) : 0;
  float* part = nullptr;
  if (pbytes) {
    void* p = nullptr;
    int rc = mlxq::workspace(pbytes, &p, s);
    if (rc) return rc;
    part = (float*)p;
  }
  const int KTS = (int)((KT + KS - 1) / KS);
  MLXQ_CHECK(batch * KS < 65536, "qmm: batch too large for one launch");
  dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM), (unsigned)(batch * KS));
  hipLaunchKernelGGL((qmm_tile_kernel<T, BITS, GS, BM, BN>), grid, dim3(256), 0, s, (const uint16_t*)x, (int)M,
                     (int)K, w, (const uint16_t*)scales, (const uint16_t*)biases, (int)N, bm, KS, KTS,
                     (uint32_t)(((bm.n_w * N * (K / GS)) * 2 + 3) & ~(int64_t)3), (uint16_t*)y, part);
  MLXQ_LAUNCHED("qmm_tile_kernel");
  if (KS > 1) {
    const int64_t n4 = batch * M * N / 4;
    hipLaunchKernelGGL((qmm_splitk_reduce_kernel<T>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       (const float4*)part, n4, KS, (uint2*)y);
    MLXQ_LAUNCHED("qmm_splitk_reduce_kernel");
  }
  return MLXQ_OK;
}

template <typename T, int BITS, int GS>
int launch_qmm_tile(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                    const void* biases, const BatchMap& bm, int64_t N, void* y, hipStream_t s) {
  if (M <= 32)
    return launch_qmm_tile_inst<T, BITS, GS, 32, 128>(x, batch, M, K, w, scales, biases, bm, N, y, s);
  if (M >= 128 && ((N + 127) / 128) * ((M + 127) / 128) * batch >= mlxq::device_cu_count())
    return launch_qmm_tile_inst<T, BITS, GS, 128, 128>(x, batch, M, K, w, scales, biases, bm, N, y, s);
  if (M <= 64)
    return launch_qmm_tile_inst<T, BITS, GS, 64, 128>(x, batch, M, K, w, scales, biases, bm, N, y, s);
  return launch_qmm_tile_inst<T, BITS, GS, 64, 64>(x, batch, M, K, w, scales, biases, bm, N, y, s);
}

// MLXQ_QMM_STREAM=0 (A/B tuning) keeps the tiled GEMM for the shapes the
// direct-to-LDS kernel takes by default; read on every call, so one process
// can compare the paths
int qmm_stream_override() {
  const char* e = getenv("MLXQ_QMM_STREAM");
  return e ? atoi(e) : 1;
}

template <typename T, int MB>
int launch_qmm_dma_inst(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                        const void* biases, const BatchMap& bm, int64_t N, void* y, hipStream_t s) {
  using SH = DmaShape<MB>;
  const int64_t KT = K / 128;
  const int64_t groups = (N + 63) / 64;
  const int64_t cus = mlxq::device_cu_count();
  // One workgroup fills a CU (its LDS).  Split K only when the row groups
  // leave a quarter of the CUs idle, until every CU has one, keeping at
  // least 8 K tiles per split (each split adds fp32 partial traffic).
  int KS = 1;
  const bool can_split = N % 4 == 0 && (uintptr_t)y % 8 == 0;
  if (can_split && 4 * groups * batch < 3 * cus)
    while (KS < 16 && groups * batch * KS < cus && KT / (KS * 2) >= 8) KS *= 2;
  const int ov = qmm_ks_override();
  if (ov >= 1 && ov <= 16 && (ov == 1 || can_split)) KS = ov;
  MLXQ_CHECK(batch * KS < 65536, "qmm: batch too large for one launch");
  const size_t pbytes = KS > 1 ? (size_t)KS * batch * M * N * sizeof(float) : 0;
  float* part = nullptr;
  if (pbytes) {
    void* p = nullptr;
    int rc = mlxq::workspace(pbytes, &p, s);
    if (rc) return rc;
    part = (float*)p;
  }
  const int KTS = (int)((KT + KS - 1) / KS);
  auto kern = qmm_dma_kernel<T, MB>;
  static bool raised = false;  // per instantiation
  if (!raised) {
    MLXQ_HIP(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, SH::LDS));
    raised = true;
  }
  dim3 grid((unsigned)groups, 1, (unsigned)(batch * KS));
  hipLaunchKernelGGL(kern, grid, dim3(512), SH::LDS, s, (const uint16_t*)x, (int)M, (int)K, w,
                     (const uint16_t*)scales, (const uint16_t*)biases, (int)N, bm, KS, KTS, (uint16_t*)y, part);
  MLXQ_LAUNCHED("qmm_dma_kernel");
  if (KS > 1) {
    const int64_t n4 = batch * M * N / 4;
    hipLaunchKernelGGL((qmm_splitk_reduce_kernel<T>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s,
                       (const float4*)part, n4, KS, (uint2*)y);
    MLXQ_LAUNCHED("qmm_splitk_reduce_kernel");
  }
  return MLXQ_OK;
}

template <typename T>
int launch_qmm_dma(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
                   const void* biases, const BatchMap& bm, int64_t N, void* y, hipStream_t s) {
  switch ((M + 15) / 16) {
    case 1: return launch_qmm_dma_inst<T, 1>(x, batch, M, K, w, scales, biases, bm, N, y, s);
    case 2: return launch_qmm_dma_inst<T, 2>(x, batch, M, K, w, scales, biases, bm, N, y, s);
    case 3: return launch_qmm_dma_inst<T, 3>(x, batch, M, K, w, scales, biases, bm, N, y, s);
    default: return launch_qmm_dma_inst<T, 4>(x, batch, M, K, w, scales, biases, bm, N, y, s);
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
                                                           int transpose, BatchMap bm, void* __restrict__ yv) {
  using S = typename T::storage;
  const S* x = reinterpret_cast<const S*>(xv);
  const S* scales = reinterpret_cast<const S*>(sv);
  const S* biases = reinterpret_cast<const S*>(bv);
  S* y = reinterpret_cast<S*>(yv);
  const int64_t bidx = blockIdx.z;
  int64_t xb, wb;
  bool xok, wok;
  bm.resolve(bidx, xb, xok, wb, wok);
  const int64_t mn = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (mn >= M * N) return;
  const int64_t m = mn / N, n = mn % N;
  x += xb * M * K;
  y += bidx * M * N;
  if (!xok || !wok) {  // absent x rows or weights: zeros
    Conv<T>::store(y, m * N + n, 0.f);
    return;
  }
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
  int RW;                      // weight rows a workgroup (<= 16 R)
  size_t lds;
};

// MLXQ_QMV_TPW (4, 8 or 16) overrides the tiles each wave streams,
// MLXQ_QMV_R (1 or 2) the 16-row weight tiles per workgroup.
int qmv_tpw_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_QMV_TPW");
    return e ? atoi(e) : 0;
  }();
  return v;
}
int qmv_r_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_QMV_R");
    return e ? atoi(e) : 0;
  }();
  return v;
}
// MLXQ_QMV_EVEN=0 keeps 16 rows a workgroup where fewer would even out the
// workgroups a CU.
int qmv_even_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_QMV_EVEN");
    return e ? atoi(e) : 1;
  }();
  return v;
}

bool plan_qmv(int bits, int gs, int64_t M, int64_t K, int64_t N, int64_t batch, QmvPlan* p) {
  const int tile_k = 512 / bits;
  const int qg = tile_k > gs ? tile_k / gs : 1;
  // whole groups (so 16-byte weight rows and 8-value x chunks); a last
  // partial tile and a group count that is not a multiple of 4 are handled
  // in the kernel
  if (K % gs || qg > 2) return false;
  const int64_t rows = M * qg;
  p->MB = rows <= 16 ? 1 : (rows <= 32 ? 2 : 0);
  if (!p->MB) return false;
  p->MR = (p->MB == 1 && rows <= 2) ? 2 : 4;
  const int64_t kt = (K + tile_k - 1) / tile_k;
  p->TPW = 0;
  const int ov = qmv_tpw_override();
  for (int tpw : {4, 8, 16}) {
    if ((kt + tpw - 1) / tpw <= 8 && (int64_t)tpw * tile_k / gs % 4 == 0 && (ov == 0 || ov == tpw)) {
      p->TPW = tpw;
      break;
    }
  }
  if (!p->TPW) return false;
  // two row tiles per workgroup when that still gives every CU a workgroup
  const int64_t cus = mlxq::device_cu_count();
  p->R = ((N + 31) / 32) * batch >= cus ? 2 : 1;
  if (rows <= 2 && ov == 0) {
    // One activation row: each wave's stream as long as possible while the
    // launch keeps >= 7 waves per CU and wastes <= 1/8 of its tiles on
    // clamped duplicates, then two row tiles per workgroup if the count
    // still holds (MI355X, 4-bit: x[1, 4096] @ W[14336, 4096]^T 10.1 ->
    // 9.2 us with 16 tiles a wave; the 262144 x 2816 head 101 -> 88 us with
    // 8 tiles a wave and two row tiles)
    auto waves = [&](int tpw, int r) { return ((N + 16 * r - 1) / (16 * r)) * batch * ((kt + tpw - 1) / tpw); };
    for (int tpw : {16, 8, 4}) {
      const int64_t nw = (kt + tpw - 1) / tpw;
      if (nw > 8 || (int64_t)tpw * tile_k / gs % 4 != 0 || 8 * (nw * tpw - kt) > kt) continue;
      if (tpw != 4 && waves(tpw, 1) < 7 * cus) continue;
      p->TPW = tpw;
      p->R = waves(tpw, 2) >= 7 * cus ? 2 : 1;
      break;
    }
  }
  if (qmv_r_override() == 1 || qmv_r_override() == 2) p->R = qmv_r_override();
  p->RW = 16 * p->R;
  // One matrix, one row tile a workgroup, and a workgroup count that is not
  // a whole number a CU (x[1, 4096] @ W[14336, 4096]^T: 896 tiles, 3.5 a CU --
  // the CUs that took a fourth workgroup finished last): as many rows a
  // workgroup as give a whole number a CU, down to 12 (the tile's other rows
  // are masked).  MI355X: 9.20 -> 9.04 us; the MoE gather (8 matrices) was
  // 1 % slower with it, so batches keep 16 rows.
  // Two row tiles a workgroup likewise at one MFMA row block (M <= 8 at
  // group 64: several workgroups share a CU at once), down to 24 rows (M = 4
  // up: 512 workgroups of 28 rows instead of 448 of 32, within noise).
  if ((p->R == 1 || p->MB == 1) && batch == 1 && qmv_even_override() != 0) {
    const int64_t full = 16 * p->R;
    const int64_t wgs = (N + full - 1) / full;
    if (wgs > cus && wgs % cus != 0) {
      const int64_t k = (wgs + cus - 1) / cus;  // workgroups a CU
      const int64_t rw = (N + k * cus - 1) / (k * cus);
      if (4 * rw >= 3 * full && rw < full) p->RW = (int)rw;
    }
  }
  p->NW = (int)((kt + p->TPW - 1) / p->TPW);
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
                    const void* biases, const BatchMap& bm, int64_t N, void* y, const QmvPlan& p, hipStream_t s) {
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
    MLXQ_CHECK(p.RW >= 1 && p.RW <= 16 * R, "qmv: rows per workgroup");
    dim3 grid((unsigned)((N + p.RW - 1) / p.RW), (unsigned)batch);
    hipLaunchKernelGGL(kern, grid, dim3(p.NW * 64), p.lds, s, (const uint16_t*)x, (int)M, (int)K, w,
                       (const uint16_t*)scales, (const uint16_t*)biases, (int)N, bm, p.RW, (uint16_t*)y);
    MLXQ_LAUNCHED("qmv_kernel");
    return MLXQ_OK;
  }
}

// launch_qmv's result when no qmv instance matches the plan (no error is
// set): the dispatch then takes the next kernel that accepts the shape
constexpr int QMV_NONE = -1;

template <typename T, int BITS, int GS>
int launch_qmv(const void* x, int64_t batch, int64_t M, int64_t K, const uint32_t* w, const void* scales,
               const void* biases, const BatchMap& bm, int64_t N, void* y, const QmvPlan& p, hipStream_t s) {
#define QMV_I(MBV, RV, TV, MRV, XCV)                                                                            \
  if (p.MB == MBV && p.R == RV && p.TPW == TV && p.MR == MRV && p.XC == XCV)                                    \
    return launch_qmv_inst<T, BITS, GS, MBV, RV, TV, MRV, XCV>(x, batch, M, K, w, scales, biases, bm, N, y, p, s);
  QMV_I(1, 1, 4, 2, 8) QMV_I(1, 1, 8, 2, 8) QMV_I(1, 1, 16, 2, 8) QMV_I(1, 2, 4, 2, 8) QMV_I(1, 2, 8, 2, 8)
  QMV_I(1, 2, 16, 2, 8) QMV_I(1, 1, 4, 4, 8) QMV_I(1, 1, 8, 4, 8) QMV_I(1, 1, 16, 4, 8) QMV_I(1, 2, 4, 4, 8)
  QMV_I(1, 2, 8, 4, 8) QMV_I(1, 2, 16, 4, 8) QMV_I(2, 1, 4, 4, 8) QMV_I(2, 1, 8, 4, 8) QMV_I(2, 1, 16, 4, 8)
  QMV_I(2, 2, 4, 4, 8) QMV_I(2, 2, 8, 4, 8) QMV_I(2, 2, 16, 4, 8)
  // larger x slices (e.g. M = 4 at K = 14336, M = 16 at K = 4096)
  QMV_I(1, 1, 16, 4, 16) QMV_I(1, 2, 16, 4, 16) QMV_I(1, 1, 8, 4, 16) QMV_I(1, 2, 8, 4, 16)
  QMV_I(2, 1, 4, 4, 16) QMV_I(2, 2, 4, 4, 16) QMV_I(2, 1, 8, 4, 16) QMV_I(2, 2, 8, 4, 16)
#undef QMV_I
  return QMV_NONE;
}

// Kernel choice shared by quantized_matmul and gather_qmm: qmv for small M,
// the tiled MFMA GEMM for larger M, the VALU kernel for everything else.
int qmm_dispatch(const void* x, int dtype, int64_t batch, int64_t M, int64_t K, const uint32_t* w,
                 const void* scales, const void* biases, const BatchMap& bm, int64_t N, int group_size, int bits,
                 int transpose, void* y, hipStream_t s) {
  QmvPlan plan;
  const bool qmv_ok = transpose && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                      (group_size == 64 || group_size == 128) && (uintptr_t)x % 16 == 0 &&
                      (uintptr_t)w % 16 == 0 && (uintptr_t)scales % 8 == 0 && (uintptr_t)biases % 8 == 0 &&
                      K * M < ((int64_t)1 << 30) && batch < 65536 &&
                      plan_qmv(bits, group_size, M, K, N, batch, &plan);
  if (qmv_ok) {
    int rc;
    if (dtype == MLXQ_BFLOAT16) {
      if (bits == 4)
        rc = group_size == 64 ? launch_qmv<BF16, 4, 64>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s)
                              : launch_qmv<BF16, 4, 128>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s);
      else
        rc = group_size == 64 ? launch_qmv<BF16, 8, 64>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s)
                              : launch_qmv<BF16, 8, 128>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s);
    } else if (bits == 4) {
      rc = group_size == 64 ? launch_qmv<F16, 4, 64>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s)
                            : launch_qmv<F16, 4, 128>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s);
    } else {
      rc = group_size == 64 ? launch_qmv<F16, 8, 64>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s)
                            : launch_qmv<F16, 8, 128>(x, batch, M, K, w, scales, biases, bm, N, y, plan, s);
    }
    if (rc != QMV_NONE) return rc;
  }

  // 4-bit group 64, M <= 64 (the shapes qmv does not take): the
  // direct-to-LDS pipelined MFMA GEMM
  const bool dma_ok = qmm_stream_override() != 0 && transpose && mlxq::is_half_dtype(dtype) && bits == 4 &&
                      group_size == 64 && K % 128 == 0 && K >= 512 && M >= 1 && M <= 64 &&
                      (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)scales % 4 == 0 &&
                      (uintptr_t)biases % 4 == 0 && 64 * K * 2 < ((int64_t)1 << 31) &&
                      N * K / 2 < ((int64_t)1 << 31) && bm.n_w * N * (K / group_size) * 2 < ((int64_t)1 << 31) &&
                      bm.seg == nullptr;
  if (dma_ok)
    return dtype == MLXQ_BFLOAT16 ? launch_qmm_dma<BF16>(x, batch, M, K, w, scales, biases, bm, N, y, s)
                                  : launch_qmm_dma<F16>(x, batch, M, K, w, scales, biases, bm, N, y, s);

  const bool tile_ok = transpose && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) && K % 64 == 0 &&
                       (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)scales % 4 == 0 &&
                       (uintptr_t)biases % 4 == 0 && M * K * 2 < ((int64_t)1 << 31) &&
                       N * K < ((int64_t)1 << 31) && bm.n_w * N * (K / group_size) * 2 < ((int64_t)1 << 31);
  if (tile_ok) {
#define QMM_TILE_T(TT)                                                                                           \
  switch (bits * 1000 + group_size) {                                                                           \
    case 4032: return launch_qmm_tile<TT, 4, 32>(x, batch, M, K, w, scales, biases, bm, N, y, s);               \
    case 4064: return launch_qmm_tile<TT, 4, 64>(x, batch, M, K, w, scales, biases, bm, N, y, s);               \
    case 4128: return launch_qmm_tile<TT, 4, 128>(x, batch, M, K, w, scales, biases, bm, N, y, s);              \
    case 8032: return launch_qmm_tile<TT, 8, 32>(x, batch, M, K, w, scales, biases, bm, N, y, s);               \
    case 8064: return launch_qmm_tile<TT, 8, 64>(x, batch, M, K, w, scales, biases, bm, N, y, s);               \
    default: return launch_qmm_tile<TT, 8, 128>(x, batch, M, K, w, scales, biases, bm, N, y, s);                \
  }
    if (dtype == MLXQ_BFLOAT16) {
      QMM_TILE_T(BF16)
    } else {
      QMM_TILE_T(F16)
    }
#undef QMM_TILE_T
  }

  const int64_t outs = M * N;
  MLXQ_CHECK(outs <= (int64_t)0x7fffffff * 256, "output too large");
  MLXQ_CHECK(batch < 65536, "batch too large for one launch");
  dim3 grid((unsigned)((outs + 255) / 256), 1, (unsigned)batch);
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 2>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, bm, y);
        break;
      case 4:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 4>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, bm, y);
        break;
      default:
        hipLaunchKernelGGL((qmm_generic_kernel<TT, 8>), grid, dim3(256), 0, s, x, M, K, w, scales, biases, N,
                           group_size, transpose, bm, y);
        break;
    }
  });
  MLXQ_LAUNCHED("qmm_generic_kernel");
  return MLXQ_OK;
}

}  // namespace

// Argument checks both entry points share.
#define QMM_COMMON_CHECKS()                                                                                  \
  MLXQ_REQUIRE_INIT();                                                                                       \
  MLXQ_CHECK(mlxq::dtype_supported(dtype), "dtype must be float16, bfloat16 or float32");                    \
  MLXQ_CHECK(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");                                 \
  MLXQ_CHECK(group_size == 32 || group_size == 64 || group_size == 128, "group_size must be 32, 64 or 128"); \
  MLXQ_CHECK(batch >= 0 && M >= 0 && K >= 0 && N >= 0, "negative extent");                                   \
  MLXQ_CHECK((transpose ? K : N) % group_size == 0, "the quantized axis must be a multiple of group_size")

extern "C" int mlxq_quantized_matmul(const void* x, int dtype, int64_t batch, int64_t M, int64_t K,
                                     const uint32_t* w, const void* scales, const void* biases, int64_t w_batch,
                                     int64_t N, int group_size, int bits, int transpose, void* y, void* stream) {
  QMM_COMMON_CHECKS();
  MLXQ_CHECK(w_batch >= 1 && batch % w_batch == 0, "batch must be a multiple of w_batch");
  if (batch == 0 || M == 0 || N == 0) return MLXQ_OK;
  MLXQ_CHECK(x && w && scales && biases && y, "null buffer");
  hipStream_t s = mlxq::resolve_stream(stream);
  if (K == 0) return mlxq_fill_zero(y, (uint64_t)(batch * M * N * mlxq::dtype_bytes(dtype)), stream);
  const BatchMap bm{nullptr, nullptr, batch, w_batch, batch / w_batch};
  return qmm_dispatch(x, dtype, batch, M, K, w, scales, biases, bm, N, group_size, bits, transpose, y, s);
}

// Sorted gather: rows of equal consecutive expert index run as one GEMM
// block (<= BM rows) of the tiled kernel, so each expert's weights stream
// once per block instead of once per row.
template <typename T, int BITS, int GS, int BM>
int launch_qmm_sorted_inst(const void* x, int64_t R, int64_t K, const uint32_t* w, const void* scales,
                           const void* biases, const uint32_t* idx, int64_t n_experts, int64_t N, void* y,
                           hipStream_t s) {
  static_assert(BM >= 1 && BM <= 128, "work-list block rows");
  void* p = nullptr;
  int rc = mlxq::workspace((1 + 3 * (size_t)R) * sizeof(int32_t), &p, s);
  if (rc) return rc;
  int32_t* seg = (int32_t*)p;
  hipLaunchKernelGGL(qmm_segments_kernel, dim3(1), dim3(1024), 0, s, idx, (int)R, BM, seg);
  MLXQ_LAUNCHED("qmm_segments_kernel");
  // sorted rows give at most R / BM + (experts present) items; a longer list
  // (unsorted rows) is walked by the same workgroups
  const int64_t slots = std::min<int64_t>(std::min<int64_t>(R, (R + BM - 1) / BM + n_experts), 65535);
  BatchMap bm{nullptr, idx, R, n_experts, 1, seg};
  dim3 grid((unsigned)((N + 127) / 128), 1, (unsigned)slots);
  hipLaunchKernelGGL((qmm_tile_kernel<T, BITS, GS, BM, 128, true>), grid, dim3(256), 0, s, (const uint16_t*)x, 1,
                     (int)K, w, (const uint16_t*)scales, (const uint16_t*)biases, (int)N, bm, 1, (int)(K / 64),
                     (uint32_t)(((n_experts * N * (K / GS)) * 2 + 3) & ~(int64_t)3), (uint16_t*)y, nullptr);
  MLXQ_LAUNCHED("qmm_tile_kernel");
  return MLXQ_OK;
}

template <typename T, int BITS, int GS>
int launch_qmm_sorted(const void* x, int64_t R, int64_t K, const uint32_t* w, const void* scales, const void* biases,
                      const uint32_t* idx, int64_t n_experts, int64_t N, void* y, hipStream_t s) {
  if (R >= 48 * n_experts)
    return launch_qmm_sorted_inst<T, BITS, GS, 64>(x, R, K, w, scales, biases, idx, n_experts, N, y, s);
  return launch_qmm_sorted_inst<T, BITS, GS, 32>(x, R, K, w, scales, biases, idx, n_experts, N, y, s);
}

extern "C" int mlxq_gather_qmm_sorted(const void* x, int dtype, int64_t rows, int64_t K, const uint32_t* rhs_indices,
                                      const uint32_t* w, const void* scales, const void* biases, int64_t n_experts,
                                      int64_t N, int group_size, int bits, void* y, void* stream) {
  const int64_t batch = rows, M = 1;
  const int transpose = 1;
  QMM_COMMON_CHECKS();
  MLXQ_CHECK(n_experts >= 1, "n_experts must be >= 1");
  MLXQ_CHECK(rows <= 0x7fffffff, "too many rows");
  if (rows == 0 || N == 0) return MLXQ_OK;
  MLXQ_CHECK(x && w && scales && biases && y && rhs_indices, "null buffer");
  hipStream_t s = mlxq::resolve_stream(stream);
  if (K == 0) return mlxq_fill_zero(y, (uint64_t)(rows * N * mlxq::dtype_bytes(dtype)), stream);
  const bool seg_ok = rows >= 2 * n_experts && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                      K % 64 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 &&
                      (uintptr_t)scales % 4 == 0 && (uintptr_t)biases % 4 == 0 && 64 * K * 2 < ((int64_t)1 << 31) &&
                      N * K < ((int64_t)1 << 31) && n_experts * N * (K / group_size) * 2 < ((int64_t)1 << 31);
  if (seg_ok) {
#define QMM_SORTED_T(TT)                                                                                         \
  switch (bits * 1000 + group_size) {                                                                           \
    case 4032: return launch_qmm_sorted<TT, 4, 32>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
    case 4064: return launch_qmm_sorted<TT, 4, 64>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
    case 4128: return launch_qmm_sorted<TT, 4, 128>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
    case 8032: return launch_qmm_sorted<TT, 8, 32>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
    case 8064: return launch_qmm_sorted<TT, 8, 64>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
    default: return launch_qmm_sorted<TT, 8, 128>(x, rows, K, w, scales, biases, rhs_indices, n_experts, N, y, s); \
  }
    if (dtype == MLXQ_BFLOAT16) {
      QMM_SORTED_T(BF16)
    } else {
      QMM_SORTED_T(F16)
    }
#undef QMM_SORTED_T
  }
  // few rows a expert (or a layout the tiled kernel does not take): one row
  // per batch element, as the unsorted gather
  const BatchMap bm{nullptr, rhs_indices, rows, n_experts, 1};
  return qmm_dispatch(x, dtype, rows, 1, K, w, scales, biases, bm, N, group_size, bits, 1, y, s);
}

extern "C" int mlxq_gather_qmm(const void* x, int dtype, int64_t x_batch, int64_t batch, int64_t M, int64_t K,
                               const int32_t* x_map, const uint32_t* rhs_indices, const uint32_t* w,
                               const void* scales, const void* biases, int64_t n_experts, int64_t N,
                               int group_size, int bits, int transpose, void* y, void* stream) {
  QMM_COMMON_CHECKS();
  MLXQ_CHECK(x_batch >= 0 && n_experts >= 1, "x_batch must be >= 0 and n_experts >= 1");
  MLXQ_CHECK(x_map || x_batch == batch, "without x_map, x_batch must equal batch");
  if (batch == 0 || M == 0 || N == 0) return MLXQ_OK;
  MLXQ_CHECK(x && w && scales && biases && y && rhs_indices, "null buffer");
  hipStream_t s = mlxq::resolve_stream(stream);
  if (K == 0) return mlxq_fill_zero(y, (uint64_t)(batch * M * N * mlxq::dtype_bytes(dtype)), stream);
  const BatchMap bm{x_map, rhs_indices, x_batch, n_experts, 1};
  return qmm_dispatch(x, dtype, batch, M, K, w, scales, biases, bm, N, group_size, bits, transpose, y, s);
}
