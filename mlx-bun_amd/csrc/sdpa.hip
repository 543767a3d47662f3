// sdpa.hip -- scaled-dot-product attention over an MLX-affine-quantized KV
// cache (gfx950): the quantizedSdpa dispatch of
// src/model/gemma4-base.ts:1560-1578 as one C entry point.
//
// Decode (Lq = 1) is HBM-bound: every K/V code, scale and bias byte is read
// once.  One workgroup owns a chunk of keys of one (batch row, kv head) and
// serves all nRep query heads of that kv head, so GQA costs no extra reads.
// Inside a wave, 32 keys at a time:
//   scores  = v_mfma 16x16x32 (A = K codes as exact operands, B = q'), with
//             the MFMA's 16 columns indexed by (quant group g, head h): the q'
//             operand of column (g, h) is head h masked to group g's
//             dimensions, so each quant group keeps its own partial dot and
//             its scale/bias are applied per key afterwards;
//   softmax = online, fp32, in the score layout (max/sum over 8 keys in
//             lane plus two cross-lane-group shuffles);
//   out    += v_mfma (A = p * s_v rounded to T, rows (g, h); B = V codes) --
//             the score layout of lane l (column l%16, keys 4*(l/16)+i and
//             16+4*(l/16)+i) is exactly the A operand layout, so p never
//             moves between lanes.
// Waves merge through LDS; the chunks of one (b, kv head) write fp32
// partials (U, M, L) that a second kernel, sdpa_decode_merge_kernel, merges
// in fixed chunk order (deterministic, no atomics).  Key chunk geometry
// handles the rotating caches' ring (slot = (ring_off - valid + j) mod cap).
//
// Everything the MFMA decode kernel does not cover (Lq > 1, D = 512 or
// nRep * D/gs > 16, 2-bit, fp32) runs a generic VALU kernel with the same
// semantics.
#include <cstdlib>
#include <initializer_list>

#include "mfma_common.h"

namespace {

constexpr float LOG2E = 1.4426950408889634f;

struct Geometry {
  int64_t cap;
  int64_t n_kv;
  const int32_t* valid_len;
  const int32_t* ring_off;
};

__device__ __forceinline__ int64_t row_valid(const Geometry& g, int b) {
  if (!g.valid_len) return g.n_kv;
  int64_t v = g.valid_len[b];
  v = v < 0 ? 0 : v;
  return v < g.cap ? v : g.cap;
}

// first physical slot of row b's logical window
__device__ __forceinline__ int64_t row_base_slot(const Geometry& g, int b, int64_t valid) {
  if (!g.ring_off) return 0;
  // (ring_off - valid) mod cap with at most one 32-bit remainder: an int32
  // offset is its own remainder once cap >= 2^31
  const int32_t r = g.ring_off[b];
  const int64_t rm = g.cap < ((int64_t)1 << 31) ? (int64_t)(r % (int32_t)g.cap) : (int64_t)r;  // |rm| < cap
  int64_t s = rm - valid;  // in (-2 cap, cap)
  s = s < 0 ? s + g.cap : s;
  return s < 0 ? s + g.cap : s;
}

__device__ __forceinline__ int64_t slot_of(int64_t base, int64_t j, int64_t cap) {
  int64_t s = base + j;
  return s >= cap ? s - cap : s;
}

// q' = T(q * T(scale)) (the reference multiplies q by the scale in T before
// the score matmul, skipping the multiply when scale == 1)
template <typename T>
__device__ __forceinline__ float scaled_q(float qv, float scale_t, bool apply) {
  return apply ? Conv<T>::round(qv * scale_t) : qv;
}

// ============================================================ MFMA decode

template <int G>
__device__ __forceinline__ uint16_t group_bits(const uint32_t (&o)[(G + 1) / 2], int g) {
  return (uint16_t)(o[g >> 1] >> (16 * (g & 1)));
}

// One cache row's G group scales (or biases): 2G contiguous bytes.
template <int G, int AUX = 0>
__device__ __forceinline__ void load_row_groups_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                    uint32_t (&o)[(G + 1) / 2]) {
  if constexpr (G == 1) {
    o[0] = __builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, AUX);
  } else if constexpr (G == 2) {
    o[0] = __builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, AUX);
  } else if constexpr (G == 4) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, AUX);
    o[0] = v[0];
    o[1] = v[1];
  } else {
    const u32x4_t v = buf_load128<AUX>(r, voff, soff);
    o[0] = v.x;
    o[1] = v.y;
    o[2] = v.z;
    o[3] = v.w;
  }
}

// Sum over the G adjacent lanes (G-aligned) that hold the G quant-group
// parts of one head's score: DPP quad permutes for G <= 4 (no LDS trip),
// every lane of the group gets the same total.
template <int G>
__device__ __forceinline__ float group_lane_sum(float v) {
  if constexpr (G >= 2)
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));  // quad_perm [1,0,3,2]
  if constexpr (G >= 4)
    v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));  // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += __shfl_xor(v, 4);
  return v;
}

// Key chunks of one batch row.  Chunk boundaries fall on multiples of
// `chunk` counted from the point where the row's logical window wraps to
// slot 0 of the ring, so every chunk occupies contiguous slots: chunk c
// covers logical keys [j0, j0 + nk) at slots [slot0, slot0 + nk).  A row
// attends nch chunks (at most ceil(valid / chunk) + 1).
struct ChunkRange {
  int64_t j0, slot0;
  int nk, nch;
};

// `chunk` is a power of two (the launchers only halve it from one), so the
// divisions are shifts: 64-bit division would expand to a few hundred
// instructions ahead of every workgroup's first load.
// A ring row whose window fills the ring attends every slot, and a decode
// chunk's keys may come in any order (softmax and the chunk merge do not
// depend on it), so such a row is cut at physical slots: ceil(cap / chunk)
// whole chunks instead of a short leading chunk, whole chunks and a short
// trailing one (one workgroup less per row when the write index is not
// chunk-aligned).
__device__ __forceinline__ ChunkRange chunk_range(const Geometry& geo, int b, int chunk, int c) {
  ChunkRange r;
  const int sh = __builtin_ctz((unsigned)chunk);
  const int64_t cm = chunk - 1;
  const int64_t valid = row_valid(geo, b);
  if (geo.ring_off && valid == geo.cap) {
    r.nch = (int)((geo.cap + cm) >> sh);
    r.j0 = r.slot0 = (int64_t)c * chunk;
    r.nk = (int)min((int64_t)chunk, geo.cap - r.slot0);
    return r;
  }
  const int64_t base = row_base_slot(geo, b, valid);  // in [0, cap)
  const int64_t jw = geo.cap - base;                  // first logical key stored at slot 0
  const int64_t off = jw < valid ? (jw & cm) : 0;     // length of a leading short chunk (0: none)
  r.nch = valid == 0 ? 0 : (off == 0 ? (int)((valid + cm) >> sh) : 1 + (int)((valid - off + cm) >> sh));
  r.j0 = off == 0 ? (int64_t)c * chunk : (c == 0 ? 0 : off + (int64_t)(c - 1) * chunk);
  const int64_t end = (off != 0 && c == 0) ? off : min(r.j0 + chunk, valid);
  r.nk = (int)(end - r.j0);
  int64_t s = base + r.j0;
  r.slot0 = s >= geo.cap ? s - geo.cap : s;
  return r;
}

// Cross-lane reductions over the four 16-lane rows of a wave (the lanes that
// hold the same MFMA column): v_permlane{16,32}_swap exchange rows in VALU.
__device__ __forceinline__ float xrow_max(float v) {
  const uint32_t u = __float_as_uint(v);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const uint32_t w = __float_as_uint(v);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xrow_sum(float v) {
  const uint32_t u = __float_as_uint(v);
  auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const uint32_t w = __float_as_uint(v);
  auto b = __builtin_amdgcn_permlane16_swap(w, w, false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Code tiles each decode wave keeps in flight (registers: WIN * KW words).
#ifndef MLXQ_DECODE_WINDOW
#define MLXQ_DECODE_WINDOW 2
#endif

// Decode tile geometry for one (T, BITS, D, GS) instance with NWV waves a
// workgroup.  The chunk (MAXC keys) does not depend on NWV: 4 waves take
// twice the tiles of 8.
template <int BITS, int D, int GS, int NWV = 8>
struct DecodeShape {
  static constexpr int NW = NWV;             // waves per workgroup
  static constexpr int KW = D * BITS / 32;   // packed words per cache row
  static constexpr int G = D / GS;
  // tiles (32 keys) per wave: up to 1024/KW a workgroup, with the chunk's
  // fp32 scales/biases (16 G bytes per key) held to 32 KB of LDS, 64 KB from
  // 4 groups a row on (D 256 at group 64: 4 tiles a wave of 8 instead of 2,
  // half the chunks; the 32-row batched ring decode 102 -> 86 us on MI355X)
  static constexpr int TPW_REG = 1024 / (KW * NW);
  static constexpr int TPW_LDS = (G >= 4 ? 4096 : 2048) / (G * NW * 32);
  static constexpr int TPW = TPW_REG < TPW_LDS ? TPW_REG : TPW_LDS;
  static constexpr int MAXC = NW * 32 * TPW;  // keys per workgroup
  static constexpr int WIN = MLXQ_DECODE_WINDOW;  // tiles in flight per wave
  // Lazy softmax rescale: the running max moves only when a tile exceeds it
  // by more than LAZY (log2 units).  At 4 groups a row with 4 tiles a wave
  // the lazy rule (p up to 2^8) widened the error tail at scale 1 (32-row
  // ring decode, D 256: 44 outputs past 0.01 against 1 with eager
  // rescaling), so those instances rescale on every new max; at D 128 both
  // rules measure the same error (scale 1 and 1/sqrt(128)) and lazy is
  // 0.4 us faster on the 32k decode.
  static constexpr float LAZY = G >= 4 ? 0.0f : 8.0f;
};

// One workgroup = NW waves = one chunk of up to MAXC keys of one (batch row,
// kv head).  NW = 8, or 4 where a launch has several workgroups a CU and
// the kernel needs more than 128 VGPRs: two 4-wave workgroups then share a
// CU where only one 8-wave workgroup would fit, so one streams while the
// other starts or finishes.  Wave w owns the 32-key tiles w + NW t,
// t < TPW.  Each wave loads its own tiles' scales/biases first and stages
// them in its LDS region as fp32 (per-key constants folded in once per key,
// not once per MFMA column; no workgroup barrier, so a wave starts on its
// first tile as soon as its own data is in); codes stream through a
// WIN-tile register window: tile t + WIN is requested as soon as tile t is
// consumed.
template <typename T, int BITS, int D, int GS, int NWV>
__global__ void __launch_bounds__(NWV * 64, 2) sdpa_decode_mfma_kernel(
    const uint16_t* __restrict__ q, const uint32_t* __restrict__ kp, const uint16_t* __restrict__ ksc,
    const uint16_t* __restrict__ kbi, const uint32_t* __restrict__ vp, const uint16_t* __restrict__ vsc,
    const uint16_t* __restrict__ vbi, int Hq, int Hkv, Geometry geo, float scale, int chunk,
    uint16_t* __restrict__ out, float* __restrict__ part_o, float2* __restrict__ part_ml) {
  using CO = CodeOps<T, BITS>;
  using SH = DecodeShape<BITS, D, GS, NWV>;
  constexpr int NW = SH::NW, TPW = SH::TPW, G = SH::G, KW = SH::KW, WIN = SH::WIN;
  constexpr int NT = NW * 64;
  constexpr int GW = (G + 1) / 2;    // dwords holding one row's G group values
  constexpr int LKW = KW / 4;        // K-side words per lane (a quarter row)
  constexpr int WPS = BITS / 4;      // K-side words per k-step
  constexpr int KSTEPS = D / 32;
  constexpr int VM = KW / 16;        // V-side word columns per lane
  constexpr int E = 32 / BITS;       // codes per word
  constexpr int DT = D / 16;         // V-side MFMA tiles
  constexpr int UMAX = 16 * GS;      // nrep * D <= 16 * GS
  constexpr float OFF = CO::OFFSET;  // code operands carry +OFF (K and V alike)
  static_assert(VM * E == DT, "tile bookkeeping");
  static_assert(LKW % 4 == 0, "K quarter rows are whole dwordx4 loads");
  static_assert(NT == NWV * 64, "launch bounds");

  // sb_lds[wave]: [0] K scale * log2e, [1] (K bias - OFF * K scale) * log2e,
  // [2] V scale, [3] V bias -- per group, for the wave's own keys (tile t at
  // 32 t): each wave stages and reads only its region, so no workgroup
  // barrier stands before its first tile.  After the tile loop the same LDS
  // holds u_lds, the per-wave unnormalised outputs [wave][h*D + d].
  constexpr int SBW = TPW * 32;  // keys per wave
  constexpr int SB_FLOATS = NW * 4 * G * SBW, U_FLOATS = NW * UMAX;
  __shared__ float lds_raw[SB_FLOATS > U_FLOATS ? SB_FLOATS : U_FLOATS];
  __shared__ float m_lds[NW][16], l_lds[NW][16];
  float(&sb_lds)[NW][4][G][SBW] = *reinterpret_cast<float(*)[NW][4][G][SBW]>(lds_raw);
  float(&u_lds)[NW][UMAX] = *reinterpret_cast<float(*)[NW][UMAX]>(lds_raw);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int b = blockIdx.z, kvh = blockIdx.y, c = blockIdx.x;
  const int nrep = Hq / Hkv;
  const int R = nrep * G;

  const ChunkRange cr = chunk_range(geo, b, chunk, c);
  const int64_t out_base = ((int64_t)b * Hq + (int64_t)kvh * nrep) * D;
  if (cr.nch == 0) {  // nothing to attend: zeros
    if (c == 0)
      for (int i = tid; i < nrep * D; i += NT) out[out_base + i] = 0;
    return;
  }
  if (c >= cr.nch) return;
  const int nk = cr.nk;

  // ---- q' operand (B of the score MFMA) -----------------------------------
  // column ln = h * G + g: a head's G group parts sit in adjacent lanes
  const int r_me = ln;
  const bool r_ok = r_me < R;
  const int g_me = r_me % G;
  const int h_me = r_ok ? r_me / G : 0;
  const float scale_t = Conv<T>::round(scale);
  const bool apply_scale = scale != 1.0f;
  u32x4_t qraw[KSTEPS];
  const uint16_t* qrow = q + out_base + (int64_t)h_me * D;
#pragma unroll
  for (int j = 0; j < KSTEPS; j++) qraw[j] = *reinterpret_cast<const u32x4_t*>(qrow + lg * (D / 4) + 8 * j);

  // ---- loads --------------------------------------------------------------
  // Raw buffer loads whose descriptors start at the chunk's first slot and
  // end after its last valid key: every load is a lane constant plus a
  // scalar offset, and keys past the chunk read 0 without touching memory
  // (their scores are masked below; zero scales/biases keep them finite).
  const int64_t row0 = ((int64_t)b * Hkv + kvh) * geo.cap + cr.slot0;
  const uint32_t nk32 = (uint32_t)nk;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp + row0 * KW, nk32 * (uint32_t)(KW * 4));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp + row0 * KW, nk32 * (uint32_t)(KW * 4));
  const __amdgpu_buffer_rsrc_t rsb[4] = {make_rsrc(ksc + row0 * G, nk32 * (uint32_t)(2 * G)),
                                         make_rsrc(kbi + row0 * G, nk32 * (uint32_t)(2 * G)),
                                         make_rsrc(vsc + row0 * G, nk32 * (uint32_t)(2 * G)),
                                         make_rsrc(vbi + row0 * G, nk32 * (uint32_t)(2 * G))};
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // this wave's scales/biases: lane l takes key l % 32 of tiles 2p + l / 32
  // (all four arrays; lanes without a tile read past the descriptors: 0)
  constexpr int SBP = (TPW + 1) / 2;  // tile pairs
  const int skey = lane & 31, shalf = lane >> 5;
  uint32_t sbreg[SBP][4][GW];
#pragma unroll
  for (int p = 0; p < SBP; p++) {
    const int t = 2 * p + shalf;
    const uint32_t voff = t < TPW ? (uint32_t)((wave_u + NW * t) * 32 + skey) * (2 * G) : 0x80000000u;
#pragma unroll
    for (int a = 0; a < 4; a++) load_row_groups_buf<G, LOAD_STREAM>(rsb[a], voff, 0u, sbreg[p][a]);
  }
  __builtin_amdgcn_sched_barrier(0);  // issue order: scales/biases, then codes

  uint32_t kbuf[WIN][2][LKW];  // [window slot][16-key sub-tile][words]
  uint32_t vbuf[WIN][8][VM];   // [window slot][key e][word column]
  // key e of a lane: e<4 -> kt + 4lg + e, e>=4 -> kt + 16 + 4lg + (e-4)
  auto issue = [&](int t, uint32_t (&kb)[2][LKW], uint32_t (&vb)[8][VM]) {
    const uint32_t kt = (uint32_t)((wave_u + NW * t) * 32);
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      const uint32_t voff = (uint32_t)(ln * KW + lg * LKW) * 4u;
      const uint32_t soff = (kt + 16u * sub) * (uint32_t)(KW * 4);
#pragma unroll
      for (int w4 = 0; w4 < LKW; w4 += 4) {
        const u32x4_t v = buf_load128<LOAD_STREAM>(rk, voff + 4u * w4, soff);
        kb[sub][w4] = v.x;
        kb[sub][w4 + 1] = v.y;
        kb[sub][w4 + 2] = v.z;
        kb[sub][w4 + 3] = v.w;
      }
    }
    // lane ln takes words VM ln .. VM ln + VM - 1 of each of its 8 keys:
    // one load per key, and 16 lanes cover whole cache rows
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t koff = (uint32_t)(e < 4 ? 4 * lg + e : 16 + 4 * lg + (e - 4));
      const uint32_t voff = (koff * KW + VM * ln) * 4u;
      const uint32_t soff = kt * (uint32_t)(KW * 4);
      if constexpr (VM == 1) {
        vb[e][0] = buf_load32<LOAD_STREAM>(rv, voff, soff);
      } else if constexpr (VM == 2) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rv, (int)voff, (int)soff, LOAD_STREAM);
        vb[e][0] = v[0];
        vb[e][1] = v[1];
      } else {
        const u32x4_t v = buf_load128<LOAD_STREAM>(rv, voff, soff);
        vb[e][0] = v.x;
        vb[e][1] = v.y;
        vb[e][2] = v.z;
        vb[e][3] = v.w;
      }
    }
  };
#pragma unroll
  for (int t = 0; t < WIN && t < TPW; t++) issue(t, kbuf[t], vbuf[t]);
  __builtin_amdgcn_sched_barrier(0);  // the window is in flight before the first wait

  // ---- stage this wave's scales/biases (fp32, per-key constants folded in)
#pragma unroll
  for (int p = 0; p < SBP; p++) {
    const int t = 2 * p + shalf;
    if (TPW % 2 == 0 || t < TPW) {
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float ks = Conv<T>::from_bits(group_bits<G>(sbreg[p][0], g));
        const float kb = Conv<T>::from_bits(group_bits<G>(sbreg[p][1], g));
        sb_lds[wave_u][0][g][32 * t + skey] = ks * LOG2E;
        sb_lds[wave_u][1][g][32 * t + skey] = (kb - OFF * ks) * LOG2E;
        sb_lds[wave_u][2][g][32 * t + skey] = Conv<T>::from_bits(group_bits<G>(sbreg[p][2], g));
        sb_lds[wave_u][3][g][32 * t + skey] = Conv<T>::from_bits(group_bits<G>(sbreg[p][3], g));
      }
    }
  }
  u32x4_t qop[KSTEPS];
  float qsum = 0.f;
#pragma unroll
  for (int j = 0; j < KSTEPS; j++) {
    const int d0 = lg * (D / 4) + 8 * j;
    const bool in_group = r_ok && (d0 / GS == g_me);
    uint32_t wv[4] = {qraw[j].x, qraw[j].y, qraw[j].z, qraw[j].w};
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const float lo = scaled_q<T>(Conv<T>::from_bits(wv[p] & 0xffffu), scale_t, apply_scale);
      const float hi = scaled_q<T>(Conv<T>::from_bits(wv[p] >> 16), scale_t, apply_scale);
      wv[p] = in_group ? Mma<T>::pack2(lo, hi) : 0u;
      qsum += in_group ? lo + hi : 0.f;
    }
    qop[j] = permute8<CO::ORDER>(u32x4_t{wv[0], wv[1], wv[2], wv[3]});
  }
  qsum = xrow_sum(qsum);
  const uint32_t magic = opaque(Mma<T>::MAGIC);
  const u32x4_t ones = {Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES, Mma<T>::ONES};

  // ---- per-wave online softmax state --------------------------------------
  float m_run = -INFINITY;  // per head h_me (log2 domain), replicated over g and lane rows
  float l_run = 0.f;        // partial over this lane's keys
  float pb_run = 0.f;       // sum of p * b_v over this lane's keys, row r_me
  f32x4_t oacc[DT];
  f32x4_t spacc = {0.f, 0.f, 0.f, 0.f};  // sum of the A operand per row (the +OFF correction)
#pragma unroll
  for (int i = 0; i < DT; i++) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int t, const uint32_t (&kb)[2][LKW], const uint32_t (&vb)[8][VM]) {
    const int kt = (wave_u + NW * t) * 32;
    const int st = 32 * t;  // this tile's keys in the wave's sb_lds region
    // scores: two 16-key sub-tiles, D/32 k-steps each
    f32x4_t sacc[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KSTEPS; j++) {
        u32x4_t a;
        if constexpr (BITS == 4)
          a = CodeOps<T, 4>::operand(kb[sub][j * WPS], magic);
        else
          a = CodeOps<T, BITS>::operand(kb[sub][j * WPS], kb[sub][j * WPS + WPS - 1]);
        acc = Mma<T>::mma(a, qop[j], acc);
      }
      sacc[sub] = acc;
    }

    float s2[8];
    {
      const float4 ka = *reinterpret_cast<const float4*>(&sb_lds[wave_u][0][g_me][st + 4 * lg]);
      const float4 kc = *reinterpret_cast<const float4*>(&sb_lds[wave_u][0][g_me][st + 16 + 4 * lg]);
      const float4 ba = *reinterpret_cast<const float4*>(&sb_lds[wave_u][1][g_me][st + 4 * lg]);
      const float4 bc = *reinterpret_cast<const float4*>(&sb_lds[wave_u][1][g_me][st + 16 + 4 * lg]);
      const float ks[8] = {ka.x, ka.y, ka.z, ka.w, kc.x, kc.y, kc.z, kc.w};
      const float kd[8] = {ba.x, ba.y, ba.z, ba.w, bc.x, bc.y, bc.z, bc.w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float cdot = e < 4 ? sacc[0][e] : sacc[1][e - 4];
        // this group's part of key e's score for head h_me (log2 domain),
        // summed over the head's G adjacent group lanes
        s2[e] = group_lane_sum<G>(__builtin_fmaf(ks[e], cdot, kd[e] * qsum));
      }
    }
    if (kt + 32 > nk) {  // the chunk's last, partial tile (wave-uniform)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int key = kt + (e < 4 ? 4 * lg + e : 12 + 4 * lg + e);
        s2[e] = key < nk ? s2[e] : -INFINITY;
      }
    }

    // online softmax over this tile's 32 keys
    float tmax = fmaxf(fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3])), fmaxf(fmaxf(s2[4], s2[5]), fmaxf(s2[6], s2[7])));
    tmax = xrow_max(tmax);
    // Lazy rescale: keep the reference max unless this tile exceeds it by
    // more than SH::LAZY (p stays <= 2^LAZY, fp32 and T both hold that
    // exactly as a scale); the accumulators are only rewritten when it moves.
    const float m_old = m_run;
    const float m_new = tmax > m_old + SH::LAZY ? tmax : m_old;  // first tile: m_old = -inf
    const float alpha = __builtin_amdgcn_exp2f(m_old - m_new);  // 1 unless moved; -inf -> 0
    m_run = m_new;
    float p[8];
#pragma unroll
    for (int e = 0; e < 8; e++) p[e] = __builtin_amdgcn_exp2f(s2[e] - m_new);
    l_run = l_run * alpha + (((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7])));

    // value-side A operand: row (h_me, g_me) = T(p * s_v); bias term in fp32
    u32x4_t aop;
    {
      const float4 sa = *reinterpret_cast<const float4*>(&sb_lds[wave_u][2][g_me][st + 4 * lg]);
      const float4 sc = *reinterpret_cast<const float4*>(&sb_lds[wave_u][2][g_me][st + 16 + 4 * lg]);
      const float4 va = *reinterpret_cast<const float4*>(&sb_lds[wave_u][3][g_me][st + 4 * lg]);
      const float4 vc = *reinterpret_cast<const float4*>(&sb_lds[wave_u][3][g_me][st + 16 + 4 * lg]);
      aop.x = Mma<T>::pack2(p[0] * sa.x, p[1] * sa.y);
      aop.y = Mma<T>::pack2(p[2] * sa.z, p[3] * sa.w);
      aop.z = Mma<T>::pack2(p[4] * sc.x, p[5] * sc.y);
      aop.w = Mma<T>::pack2(p[6] * sc.z, p[7] * sc.w);
      float pbt = p[0] * va.x;
      pbt = __builtin_fmaf(p[1], va.y, pbt);
      pbt = __builtin_fmaf(p[2], va.z, pbt);
      pbt = __builtin_fmaf(p[3], va.w, pbt);
      pbt = __builtin_fmaf(p[4], vc.x, pbt);
      pbt = __builtin_fmaf(p[5], vc.y, pbt);
      pbt = __builtin_fmaf(p[6], vc.z, pbt);
      pbt = __builtin_fmaf(p[7], vc.w, pbt);
      pb_run = __builtin_fmaf(pb_run, alpha, pbt);
    }

    // rescale the accumulator rows (4lg + i) by their head's alpha (the
    // first tile skips this: the accumulators are still zero)
    if (__any(alpha != 1.0f && m_old != -INFINITY)) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ai = __shfl(alpha, 4 * lg + i);
        spacc[i] *= ai;
#pragma unroll
        for (int tt = 0; tt < DT; tt++) oacc[tt][i] *= ai;
      }
    }
    if constexpr (OFF != 0.0f) spacc = Mma<T>::mma(aop, ones, spacc);

    // value MFMAs: tile (m, e') covers d = (VM ln + m) * E + e'
#pragma unroll
    for (int m = 0; m < VM; m++) {
      if constexpr (BITS == 4) {
        uint32_t pv[2][4];  // [lo/hi halves][key pair]
#pragma unroll
        for (int pr = 0; pr < 4; pr++) {
          pv[0][pr] = perm_b32(vb[2 * pr + 1][m], vb[2 * pr][m], 0x05040100u);
          pv[1][pr] = perm_b32(vb[2 * pr + 1][m], vb[2 * pr][m], 0x07060302u);
        }
#pragma unroll
        for (int ep = 0; ep < 8; ep++) {
          const int sh = 4 * (ep & 3);
          const uint32_t* src = pv[ep >> 2];
          const u32x4_t bop = {bfi32(0x000f000fu, src[0] >> sh, magic), bfi32(0x000f000fu, src[1] >> sh, magic),
                               bfi32(0x000f000fu, src[2] >> sh, magic), bfi32(0x000f000fu, src[3] >> sh, magic)};
          oacc[m * E + ep] = Mma<T>::mma(aop, bop, oacc[m * E + ep]);
        }
      } else {
#pragma unroll
        for (int ep = 0; ep < 4; ep++) {
          uint32_t bw[4];
#pragma unroll
          for (int pr = 0; pr < 4; pr++) {
            const uint32_t wa = vb[2 * pr][m], wb = vb[2 * pr + 1][m];
            if constexpr (std::is_same<T, BF16>::value) {
              const float fa = (float)((wa >> (8 * ep)) & 0xffu);
              const float fb = (float)((wb >> (8 * ep)) & 0xffu);
              bw[pr] = perm_b32(__float_as_uint(fb), __float_as_uint(fa), 0x07060302u);
            } else {
              // bytes [a_ep, 0, b_ep, 0] | 1024.0 f16 pair
              const uint32_t sel = (uint32_t)ep | 0x0c00u | ((uint32_t)(4 + ep) << 16) | 0x0c000000u;
              bw[pr] = perm_b32(wb, wa, sel) | 0x64006400u;
            }
          }
          oacc[m * E + ep] = Mma<T>::mma(aop, u32x4_t{bw[0], bw[1], bw[2], bw[3]}, oacc[m * E + ep]);
        }
      }
    }
  };

  // ---- stream the wave's tiles through the two-slot window ----------------
#pragma unroll
  for (int t = 0; t < TPW; t++) {
    if ((wave_u + NW * t) * 32 < nk) compute(t, kbuf[t % WIN], vbuf[t % WIN]);  // wave-uniform
    __builtin_amdgcn_sched_barrier(0);
    if (t + WIN < TPW) issue(t + WIN, kbuf[t % WIN], vbuf[t % WIN]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ---- wave result: u[h][d] = O - OFF * sp + pb (rows whose group owns d) -
  l_run = xrow_sum(l_run);
  pb_run = xrow_sum(pb_run);
  lds_barrier();  // every wave is done reading sb_lds, which u_lds overlays
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * lg + i;
    const float pb_r = __shfl(pb_run, r);
    if (r < R) {
      const int g = r % G, h = r / G;
      const float corr = pb_r - OFF * spacc[i];
#pragma unroll
      for (int tt = 0; tt < DT; tt++) {
        const int m = tt / E, ep = tt % E;
        const int d = (VM * ln + m) * E + ep;
        if (d / GS == g) u_lds[wave][h * D + d] = oacc[tt][i] + corr;
      }
    }
  }
  if (lane < R && g_me == 0) {
    m_lds[wave][h_me] = m_run;
    l_lds[wave][h_me] = l_run;
  }
  lds_barrier();

  // ---- merge the waves (fixed order) ---------------------------------------
  const bool single = cr.nch == 1;
  const int64_t bk = (int64_t)b * Hkv + kvh;
  const int nd = nrep * D;
  const int64_t pc = bk * gridDim.x + c;  // this chunk's partial slot
  for (int idx = tid; idx < nd; idx += NT) {
    const int h = idx / D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, m_lds[w][h]);
    float U = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float f = __builtin_amdgcn_exp2f(m_lds[w][h] - M);  // idle wave: m = -inf -> 0
      U = __builtin_fmaf(f, u_lds[w][idx], U);
      L = __builtin_fmaf(f, l_lds[w][h], L);
    }
    if (single) {
      Conv<T>::store(out, out_base + idx, U / L);
    } else {
      part_o[pc * nd + idx] = U;
      if (idx % D == 0) part_ml[pc * nrep + h] = make_float2(M, L);
    }
  }
}

// Split-K merge: out[b, kvh*nrep + h, d] = sum_c U_c e^{M_c - M} / sum_c L_c e^{M_c - M}
// over the chunks c of row b (the reference's deterministic flash-decoding
// merge, src/model/fused-decode-kernel.ts:205-222).  Workgroup (cb, kvh, b)
// owns 64 float4 columns of (h, d); its NWM waves (~8 chunks each, see
// launch_merge) fold the chunks c = wave, wave + NWM, ... with an online
// merge and combine in LDS in fixed order.  chunk > 0: the chunks
// are the decode chunks of row b (rows whose keys fit one chunk were
// finished by the partial kernel); chunk == 0: every row has nslots chunks
// (the split prefill, whose rows h are (head, query) pairs in output order).
// A chunk with no unmasked key (M = -inf) adds nothing; a row with none
// at all stores 0, as the single-pass kernels do.
template <typename T, int NWM>
__global__ void __launch_bounds__(NWM * 64) sdpa_decode_merge_kernel(const float4* __restrict__ part_o,
                                                                const float2* __restrict__ part_ml, int Hq, int Hkv,
                                                                int D, Geometry geo, int chunk, int nslots,
                                                                uint16_t* __restrict__ out) {
  __shared__ float4 ul[NWM][64];
  __shared__ float2 mll[NWM][64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int nw = NWM;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const int nrep = Hq / Hkv;
  const int cols = nrep * D / 4;
  const int col = blockIdx.x * 64 + lane;
  const int nch = chunk > 0 ? chunk_range(geo, b, chunk, 0).nch : nslots;
  if (chunk > 0 && nch <= 1) return;
  const int64_t bk = (int64_t)b * Hkv + kvh;
  const bool active = col < cols;
  const int colc = active ? col : cols - 1;
  const int h = (colc * 4) / D;
  const float4* po = part_o + bk * nslots * cols;
  const float2* pml = part_ml + bk * nslots * nrep;
  float M = -INFINITY, L = 0.f;
  float4 U = make_float4(0.f, 0.f, 0.f, 0.f);
  // batches of 8 chunks per wave: all 16 loads of a batch are issued before
  // any of its math (one memory round trip per batch, not one per chunk)
  for (int c0 = wave; c0 < nch; c0 += 8 * nw) {
    float2 ml[8];
    float4 u[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int cc = min(c0 + i * nw, nch - 1);  // past nch: a valid slot, not folded
      ml[i] = pml[cc * nrep + h];
      u[i] = po[(int64_t)cc * cols + colc];
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
      // a fully masked chunk (M = -inf, L = U = 0) leaves the fold as it
      // is; selects, not a branch, so the math waits on one load at a time
      const bool live = c0 + i * nw < nch && ml[i].x != -INFINITY;
      const float Mn = live ? fmaxf(M, ml[i].x) : M;
      const float a = live ? __builtin_amdgcn_exp2f(M - Mn) : 1.0f;  // M = -inf -> a = 0
      const float f = live ? __builtin_amdgcn_exp2f(ml[i].x - Mn) : 0.0f;
      L = L * a + ml[i].y * f;
      U.x = U.x * a + u[i].x * f;
      U.y = U.y * a + u[i].y * f;
      U.z = U.z * a + u[i].z * f;
      U.w = U.w * a + u[i].w * f;
      M = Mn;
    }
  }
  ul[wave][lane] = U;
  mll[wave][lane] = make_float2(M, L);
  lds_barrier();
  if (wave != 0 || !active) return;
  float Mt = -INFINITY;
#pragma unroll
  for (int w = 0; w < nw; w++) Mt = fmaxf(Mt, mll[w][lane].x);
  float Lt = 0.f;
  float4 Ut = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int w = 0; w < nw; w++) {
    const float mw = mll[w][lane].x;
    const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - Mt);  // wave with no chunk adds 0
    const float4 u = ul[w][lane];
    Lt = __builtin_fmaf(f, mll[w][lane].y, Lt);
    Ut.x = __builtin_fmaf(f, u.x, Ut.x);
    Ut.y = __builtin_fmaf(f, u.y, Ut.y);
    Ut.z = __builtin_fmaf(f, u.z, Ut.z);
    Ut.w = __builtin_fmaf(f, u.w, Ut.w);
  }
  const bool any = Lt > 0.f;
  const int64_t o = ((int64_t)b * Hq + (int64_t)kvh * nrep) * D + (int64_t)col * 4;
  Conv<T>::store(out, o, any ? Ut.x / Lt : 0.f);
  Conv<T>::store(out, o + 1, any ? Ut.y / Lt : 0.f);
  Conv<T>::store(out, o + 2, any ? Ut.z / Lt : 0.f);
  Conv<T>::store(out, o + 3, any ? Ut.w / Lt : 0.f);
}

// Merge of up to nslots chunks per row: ~8 chunks a wave (the fold's
// unroll), 2 to 16 waves.
template <typename T>
int launch_merge(dim3 grid, int64_t nslots, hipStream_t s, const float* part_o, const float2* part_ml, int Hq,
                  int Hkv, int D, Geometry geo, int chunk, uint16_t* out) {
  const int64_t want = (nslots + 7) / 8;
#define MERGE_AT(W)                                                                                              \
  hipLaunchKernelGGL((sdpa_decode_merge_kernel<T, W>), grid, dim3(64 * W), 0, s, (const float4*)part_o, part_ml, \
                     Hq, Hkv, D, geo, chunk, (int)nslots, out)
  if (want <= 2)
    MERGE_AT(2);
  else if (want <= 4)
    MERGE_AT(4);
  else if (want <= 8)
    MERGE_AT(8);
  else
    MERGE_AT(16);
#undef MERGE_AT
  MLXQ_LAUNCHED("sdpa_decode_merge_kernel");
  return MLXQ_OK;
}

// ===================================================== MFMA decode, wide rows
//
// Decode when a kv head's (head, group) pairs exceed the 16 score columns of
// the kernel above (nRep * D/gs > 16: Gemma4's full-attention layers run
// 8 query heads per kv head at head_dim 512, src/config.ts:150-156, and only
// those layers keep a quantized cache, src/model/gemma4-base.ts:414-417).
// One workgroup = 8 waves = one chunk of keys of one (batch row, kv head),
// streamed in 128-key tiles:
//   * scores S = Q K^T on v_mfma_f32_16x16x32 with the heads as rows (A = q',
//     loaded once) and 16 keys per wave as columns (B = exact code operands
//     OFF + c straight from memory).  Each K load reads 16 keys x 64
//     contiguous bytes (lane quarter lq: bytes [16 lq, 16 lq + 16) of the
//     64); a 4 x 4 dword transpose across the quarters (v_permlane32_swap,
//     v_permlane16_swap) then gives every k-step 32 consecutive codes, so
//     a k-step never leaves a group.  Per group S += s_k * D +
//     (b_k - OFF s_k) * X_g, s_k and b_k being per-lane scalars (the
//     column is the key) and X_g the head's sum of q' over the group -- no
//     rounding of the dequantized K;
//   * one tile max per head shared through LDS, P = exp2(S - m) written to
//     LDS as T, the row sum taken over the same T values;
//   * V dequantized once per tile (fp32 s * c + b -> T) into a transposed
//     LDS tile, and O += P V with each wave owning D/8 output dims (no
//     cross-wave output merge).  A staging item is one 16-byte block of 4
//     consecutive keys, so each V load instruction reads whole rows;
//     smaller loads spread over many rows cost more in request count
//     than in bytes (the memory pipeline, not HBM, was the limit);
//   * the next tile's codes and scales are requested once this one's are
//     consumed (after the score MFMAs), ahead of its softmax and P V.
// Chunks write (U, M, L) partials for sdpa_decode_merge_kernel, exactly as
// the kernel above does.
template <int D, int GS, int BITS>
struct WideShape {
  static constexpr int NW = 8;                    // waves (4 waves of 64-key tiles measured slower)
  static constexpr int TK = 16 * NW;              // keys per tile (16 per wave)
  static constexpr int G = D / GS;
  static constexpr int RB = D * BITS / 8;         // bytes per cache row
  static constexpr int KW = RB / 4;               // code words per cache row
  static constexpr int KI = RB / 64;              // K loads per lane: 16 keys x 64 bytes each
  static constexpr int NKS = D / 32;              // 16x16x32 k-steps per row
  static constexpr int KST = GS / 32;             // ... per group
  static constexpr int VTP = TK + 8;              // V^T / P row pitch (T elements)
  static constexpr int DPW = D / NW;              // output dims per wave
  static constexpr int CT = DPW / 16;             // 16-dim output column tiles per wave
  static constexpr int NDB = RB / 16;             // 16-byte blocks per row
  static constexpr int DB = 128 / BITS;           // dims per block
  static constexpr int NVI = (TK / 4) * NDB;      // V staging items (4 keys x one block)
  static constexpr int IPT = (NVI + NW * 64 - 1) / (NW * 64);
  static constexpr int GW = (G + 1) / 2;          // dwords per row of G scales
  static constexpr int MAXC = 1024;
};

// V^T column swizzle: the 8-key block cb of dim row d is stored at block
// cb ^ ((d / DB) % NB), NB = keys per tile / 8, so the lanes of one staging
// store (same dim of consecutive 16-byte blocks) spread over the LDS banks.
template <int DB, int NB>
__device__ __forceinline__ int vt_block(int d, int cb) {
  return cb ^ ((d / DB) & (NB - 1));
}

template <typename T, int BITS, int D, int GS>
__global__ void __launch_bounds__(512) sdpa_decode_wide_kernel(
    const uint16_t* __restrict__ q, const uint32_t* __restrict__ kp, const uint16_t* __restrict__ ksc,
    const uint16_t* __restrict__ kbi, const uint32_t* __restrict__ vp, const uint16_t* __restrict__ vsc,
    const uint16_t* __restrict__ vbi, int Hq, int Hkv, Geometry geo, float scale, int chunk,
    uint16_t* __restrict__ out, float* __restrict__ part_o, float2* __restrict__ part_ml) {
  using SH = WideShape<D, GS, BITS>;
  using CO = CodeOps<T, BITS>;
  constexpr int NW = SH::NW, TK = SH::TK, G = SH::G, KW = SH::KW, KI = SH::KI, NKS = SH::NKS, KST = SH::KST;
  constexpr int VTP = SH::VTP, DPW = SH::DPW, CT = SH::CT, NDB = SH::NDB, DB = SH::DB, NVI = SH::NVI;
  constexpr int IPT = SH::IPT, GW = SH::GW;
  constexpr float OFF = CO::OFFSET;
  constexpr uint32_t CMASK = (1u << BITS) - 1u;
  constexpr int NB = TK / 8;
  static_assert(G <= 8 && CT >= 1 && KI >= 1 && TK % 32 == 0, "wide decode geometry");
  __shared__ __align__(16) uint16_t vt[D * VTP];  // V^T tile, T
  __shared__ __align__(16) uint16_t pl[16 * VTP]; // P tile [head][key], T
  __shared__ float xsum[G][16];                   // X[group][head]
  __shared__ float tmx[NW][16], lsm[NW][16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lq = lane >> 4;
  const int b = blockIdx.z, kvh = blockIdx.y, c = blockIdx.x;
  const int nslots = gridDim.x;
  const int nrep = Hq / Hkv;
  const ChunkRange cr = chunk_range(geo, b, chunk, c);
  const int64_t out_base = ((int64_t)b * Hq + (int64_t)kvh * nrep) * D;
  if (cr.nch == 0) {  // nothing to attend: zeros
    if (c == 0)
      for (int i = tid; i < nrep * D; i += NW * 64) out[out_base + i] = 0;
    return;
  }
  if (c >= cr.nch) return;
  const int nk = cr.nk;
  const int ntiles = (nk + TK - 1) / TK;

  // ---- descriptors (keys past the chunk read 0) ----------------------------
  const int64_t row0 = ((int64_t)b * Hkv + kvh) * geo.cap + cr.slot0;
  const uint32_t nk32 = (uint32_t)nk;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp + row0 * KW, nk32 * (uint32_t)(KW * 4));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp + row0 * KW, nk32 * (uint32_t)(KW * 4));
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksc + row0 * G, nk32 * (uint32_t)(2 * G));
  const __amdgpu_buffer_rsrc_t rkb = make_rsrc(kbi + row0 * G, nk32 * (uint32_t)(2 * G));
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(vsc + row0 * G, nk32 * (uint32_t)(2 * G));
  const __amdgpu_buffer_rsrc_t rvb = make_rsrc(vbi + row0 * G, nk32 * (uint32_t)(2 * G));

  // K side of a tile: lane (key ln of this wave's 16, quarter lq); w[j] is
  // bytes [64 j + 16 lq, 64 j + 16 lq + 16) of the row until transposed
  struct KSlot {
    uint32_t w[KI][4];
    uint32_t s[GW], bb[GW];
  };
  // V side: item it = tid + 512 p is 16-byte block it % NDB of keys
  // 4 (it / NDB) + [0, 4); s / bb hold each key's dword with the block's group
  struct VSlot {
    uint32_t w[IPT][4][4];
    uint32_t s[IPT][4], bb[IPT][4];
  };
  auto load_k = [&](int t, KSlot& k) {
    const uint32_t key = (uint32_t)(TK * t + 16 * wave + ln);
#pragma unroll
    for (int j = 0; j < KI; j++) {
      const u32x4_t v = buf_load128<LOAD_STREAM>(rk, (key * KW + 16u * j + 4u * lq) * 4u, 0u);
      k.w[j][0] = v.x;
      k.w[j][1] = v.y;
      k.w[j][2] = v.z;
      k.w[j][3] = v.w;
    }
    load_row_groups_buf<G, LOAD_STREAM>(rks, key * (uint32_t)(2 * G), 0u, k.s);
    load_row_groups_buf<G, LOAD_STREAM>(rkb, key * (uint32_t)(2 * G), 0u, k.bb);
  };
  auto load_v = [&](int t, VSlot& v) {
#pragma unroll
    for (int p = 0; p < IPT; p++) {
      const int it = tid + NW * 64 * p;
      const bool act = it < NVI;
      const int db = it % NDB, kq = it / NDB;
      const int vg = (DB * db) / GS;
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const uint32_t key = (uint32_t)(TK * t + 4 * kq + kk);
        const uint32_t off = act ? (key * KW + 4u * db) * 4u : 0x80000000u;  // inactive: reads 0
        const u32x4_t x = buf_load128<LOAD_STREAM>(rv, off, 0u);
        v.w[p][kk][0] = x.x;
        v.w[p][kk][1] = x.y;
        v.w[p][kk][2] = x.z;
        v.w[p][kk][3] = x.w;
        const uint32_t so = act ? ((key * (uint32_t)G + (uint32_t)vg) * 2u) & ~3u : 0x80000000u;
        v.s[p][kk] = __builtin_amdgcn_raw_buffer_load_b32(rvs, (int)so, 0, LOAD_STREAM);
        v.bb[p][kk] = __builtin_amdgcn_raw_buffer_load_b32(rvb, (int)so, 0, LOAD_STREAM);
      }
    }
  };
  // V: s * c + b -> T, written as V^T rows (one per dim) of 4 keys, the key
  // blocks swizzled by vt_block
  auto stage_v = [&](int t, const VSlot& v) {
#pragma unroll
    for (int p = 0; p < IPT; p++) {
      const int it = tid + NW * 64 * p;
      if (it >= NVI) continue;
      const int db = it % NDB, kq = it / NDB;
      const int vg = (DB * db) / GS;
      float sc[4], bi[4];
#pragma unroll
      for (int kk = 0; kk < 4; kk++) {
        const int shk = 16 * (int)((((uint32_t)(TK * t + 4 * kq + kk) * (uint32_t)G + (uint32_t)vg)) & 1u);
        sc[kk] = Conv<T>::from_bits((v.s[p][kk] >> shk) & 0xffffu);
        bi[kk] = Conv<T>::from_bits((v.bb[p][kk] >> shk) & 0xffffu);
      }
      const int col = 8 * vt_block<DB, NB>(DB * db, kq >> 1) + 4 * (kq & 1);  // every dim of the block: same swizzle
#pragma unroll
      for (int e = 0; e < DB; e++) {
        float x[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const uint32_t wv = v.w[p][kk][e * BITS / 32];
          x[kk] = __builtin_fmaf(sc[kk], (float)((wv >> ((e * BITS) % 32)) & CMASK), bi[kk]);
        }
        *reinterpret_cast<uint2*>(&vt[(DB * db + e) * VTP + col]) =
            make_uint2(Mma<T>::pack2(x[0], x[1]), Mma<T>::pack2(x[2], x[3]));
      }
    }
  };

  // ---- q' (A operand) and X ------------------------------------------------
  // The nrep query rows are read once per workgroup (16 bytes a thread),
  // scaled, and staged in LDS (the V^T tile, free until the first tile is
  // staged); tile 0's code loads are issued in between so their latency
  // overlaps.  A-operand row = head ln; k-step ks covers dims
  // [32 ks, 32 ks + 32), quarter lq the dims its transposed K words carry:
  // 4-bit 32 ks + 8 lq + [0, 8), 8-bit 32 ks + 4 lq + [0, 4) then
  // 32 ks + 16 + 4 lq + [0, 4).
  constexpr int QP = D + 8;  // staged q' row pitch (T elements)
  constexpr int QIT = (16 * (D / 8) + NW * 64 - 1) / (NW * 64);
  static_assert(16 * QP <= D * VTP, "q' staging fits in the V^T tile");
  const int qitems = nrep * (D / 8);
  u32x4_t qraw[QIT];
#pragma unroll
  for (int p = 0; p < QIT; p++) {
    const int it = tid + NW * 64 * p;
    qraw[p] = it < qitems ? *reinterpret_cast<const u32x4_t*>(q + out_base + 8 * (int64_t)it) : u32x4_t{0u, 0u, 0u, 0u};
  }
  KSlot kslot;
  VSlot vslot;
  load_k(0, kslot);
  load_v(0, vslot);
  const float scale_t = Conv<T>::round(scale);
  const bool apply_scale = scale != 1.0f;
#pragma unroll
  for (int p = 0; p < QIT; p++) {
    const int it = tid + NW * 64 * p;
    if (it < qitems) {
      u32x4_t r = qraw[p];
#pragma unroll
      for (int p2 = 0; p2 < 4; p2++)
        r[p2] = Mma<T>::pack2(scaled_q<T>(Conv<T>::from_bits(r[p2] & 0xffffu), scale_t, apply_scale),
                              scaled_q<T>(Conv<T>::from_bits(r[p2] >> 16), scale_t, apply_scale));
      *reinterpret_cast<u32x4_t*>(&vt[(it / (D / 8)) * QP + 8 * (it % (D / 8))]) = r;
    }
  }
  lds_barrier();  // q' in
  const bool hok = ln < nrep;
  const uint16_t* qrow = vt + ln * QP;
  u32x4_t qop[NKS];
#pragma unroll
  for (int g = 0; g < G; g++) {
    float xp = 0.f;
#pragma unroll
    for (int s = 0; s < KST; s++) {
      const int ks = g * KST + s;
      u32x4_t raw = {0u, 0u, 0u, 0u};
      if (hok) {
        if constexpr (BITS == 4) {
          raw = *reinterpret_cast<const u32x4_t*>(qrow + 32 * ks + 8 * lq);
        } else {
          const uint2 lo = *reinterpret_cast<const uint2*>(qrow + 32 * ks + 4 * lq);
          const uint2 hi = *reinterpret_cast<const uint2*>(qrow + 32 * ks + 16 + 4 * lq);
          raw = u32x4_t{lo.x, lo.y, hi.x, hi.y};
        }
      }
#pragma unroll
      for (int p2 = 0; p2 < 4; p2++) xp += Conv<T>::from_bits(raw[p2] & 0xffffu) + Conv<T>::from_bits(raw[p2] >> 16);
      qop[ks] = permute8<CO::ORDER>(raw);
    }
    xp += __shfl_xor(xp, 16);
    xp += __shfl_xor(xp, 32);
    if (wave == 0 && lq == 0) xsum[g][ln] = xp;
  }

  // ---- online softmax state: rows 4 lq + i (heads) of the 16x16 layouts ----
  float m_run[4], l_run[4];
  f32x4_t oacc[CT];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }
#pragma unroll
  for (int ct = 0; ct < CT; ct++) oacc[ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const uint32_t magic = opaque(Mma<T>::MAGIC);

  // one register slot each: a tile consumes its codes (V staging, score
  // MFMAs) before the next tile's loads refill the same slots
  auto tile = [&](int t, KSlot& k, VSlot& v) {
    stage_v(t, v);
#pragma unroll
    for (int j = 0; j < KI; j++) quarter_transpose(k.w[j]);
    // scores of this wave's 16 keys, log2 units
    f32x4_t sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < G; g++) {
      f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KST; s++) {
        const int ks = g * KST + s;
        u32x4_t bop;
        if constexpr (BITS == 4)
          bop = CodeOps<T, 4>::operand(k.w[ks / 4][ks % 4], magic);
        else
          bop = CodeOps<T, BITS>::operand(k.w[ks / 2][2 * (ks % 2)], k.w[ks / 2][2 * (ks % 2) + 1]);
        part = Mma<T>::mma(qop[ks], bop, part);
      }
      const float ks = Conv<T>::from_bits(group_bits<G>(k.s, g));
      const float kd = (Conv<T>::from_bits(group_bits<G>(k.bb, g)) - OFF * ks) * LOG2E;
      const float4 xv = *reinterpret_cast<const float4*>(&xsum[g][4 * lq]);
      const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int i = 0; i < 4; i++) sacc[i] = __builtin_fmaf(ks * LOG2E, part[i], __builtin_fmaf(kd, xa[i], sacc[i]));
    }
    const bool key_ok = TK * t + 16 * wave + ln < nk;
    float tmax[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      sacc[i] = key_ok ? sacc[i] : -INFINITY;
      float mv = sacc[i];
      mv = fmaxf(mv, __shfl_xor(mv, 1));
      mv = fmaxf(mv, __shfl_xor(mv, 2));
      mv = fmaxf(mv, __shfl_xor(mv, 4));
      mv = fmaxf(mv, __shfl_xor(mv, 8));
      tmax[i] = mv;
    }
    if (ln == 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) tmx[wave][4 * lq + i] = tmax[i];
    }
    if (t + 1 < ntiles) {  // workgroup-uniform
      load_k(t + 1, k);
      load_v(t + 1, v);
    }
    lds_barrier();  // tile maxima and V^T in
    float alpha[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float tm = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; w++) tm = fmaxf(tm, tmx[w][4 * lq + i]);
      const float m_old = m_run[i];
      const float m_new = tm > m_old + 8.0f ? tm : m_old;  // lazy: p <= 2^8
      alpha[i] = m_new == m_old ? 1.0f : __builtin_amdgcn_exp2f(m_old - m_new);
      m_run[i] = m_new;
      const float msub = m_new == -INFINITY ? 0.f : m_new;
      const uint32_t pb = Conv<T>::to_bits(__builtin_amdgcn_exp2f(sacc[i] - msub));
      pl[(4 * lq + i) * VTP + 16 * wave + ln] = (uint16_t)pb;
      l_run[i] = l_run[i] * alpha[i] + Conv<T>::from_bits(pb);  // the P the MFMA sees
    }
    if (__any(alpha[0] != 1.0f || alpha[1] != 1.0f || alpha[2] != 1.0f || alpha[3] != 1.0f)) {
#pragma unroll
      for (int ct = 0; ct < CT; ct++)
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[ct][i] *= alpha[i];
    }
    lds_barrier();  // P in
#pragma unroll
    for (int kq = 0; kq < TK / 32; kq++) {
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&pl[ln * VTP + 32 * kq + 8 * lq]);
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const int d = DPW * wave + 16 * ct + ln;
        const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(&vt[d * VTP + 8 * vt_block<DB, NB>(d, 4 * kq + lq)]);
        oacc[ct] = Mma<T>::mma(a, bv, oacc[ct]);
      }
    }
    lds_barrier();  // the tile's V^T and P are free again
  };

  lds_barrier();  // X in; q' reads done before V^T staging
  for (int t = 0; t < ntiles; t++) tile(t, kslot, vslot);

  // ---- row sums over keys (lanes) and waves; store -------------------------
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float lv = l_run[i];
    lv += __shfl_xor(lv, 1);
    lv += __shfl_xor(lv, 2);
    lv += __shfl_xor(lv, 4);
    lv += __shfl_xor(lv, 8);
    if (ln == 0) lsm[wave][4 * lq + i] = lv;
  }
  lds_barrier();
  const bool single = cr.nch == 1;
  const int64_t pc = ((int64_t)b * Hkv + kvh) * nslots + c;  // this chunk's partial slot
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int h = 4 * lq + i;
    if (h < nrep) {
      float L = 0.f;
#pragma unroll
      for (int w = 0; w < NW; w++) L += lsm[w][h];
#pragma unroll
      for (int ct = 0; ct < CT; ct++) {
        const int d = DPW * wave + 16 * ct + ln;
        if (single)
          Conv<T>::store(out, out_base + (int64_t)h * D + d, oacc[ct][i] / L);
        else
          part_o[(pc * nrep + h) * D + d] = oacc[ct][i];
      }
      if (!single && wave == 0 && ln == 0) part_ml[pc * nrep + h] = make_float2(m_run[i], L);
    }
  }
}

// ========================================================== MFMA prefill
//
// Lq > 1 (chunked prefill over the quantized cache, quantizedSdpaTiled's
// job, src/model/gemma4-base.ts:1356-1521) is a dense contraction, so it
// runs on the matrix cores.  A workgroup owns 256 query rows of one (batch
// row, kv head): row r = (query i, head h) with r = i_local * nRep + h, so
// every head of the kv head shares each K/V tile.  Per 64-key tile:
//   * K goes to LDS as exact code operands (OFF + c as T, [key][d]) next to
//     fp32 per-key (s, b - OFF s) of every group; V is dequantized (fp32
//     s * c + b, rounded to T) and stored transposed as [d][key'] with the
//     keys of every 16-key group in the order the P operand below produces;
//   * each wave computes S^T = K Q^T for its 32 rows with
//     v_mfma_f32_32x32x16 (lane l holds column (query row) l % 32 and 16
//     keys of each 32-key block) as
//     S^T = sum_g (b - OFF s)_g X_g + sum_g s_g (C_g Q_g^T), X_g the row's
//     sum of q' over group g: the first sum is one more MFMA per block (the
//     fp32 b - OFF s and X each split exactly into three truncated bf16
//     parts, the six products down to 2^-16 of the leading one in the k
//     slots), the second a chain of code MFMAs per group folded with s in
//     fp32 -- scores carry no rounding of the dequantized K (at scale 1 and
//     |q||k| ~ 10 a T-rounded K would move them by ~1e-2); a row's softmax
//     is in-lane work plus one exchange with lane l ^ 32;
//   * online softmax in fp32 (lazy rescale), then O^T += V^T P^T where the
//     P^T operand is exactly the lane's own probabilities packed to T.
// Next tile's codes are loaded into registers while the current tile
// computes; LDS is double-buffered (one barrier per tile).  Causal / window
// masks are applied only on tiles that straddle a row's boundary.
template <int D>
struct PrefillShape {
  static constexpr int BN = 64;                   // keys per tile
  static constexpr int NW = 8;                    // waves (32 query rows each)
  static constexpr int ROWS = 32 * NW;
  static constexpr int KP = D + 8;                // K tile pitch (T elements)
  static constexpr int VP = BN + 8;               // V^T tile pitch
  static constexpr int KI = BN * D / 32;          // K items: 32 codes of one key
  static constexpr int VI = (BN / 4) * (D / 8);   // V items: 8 codes of 4 keys
  static constexpr int IPT = (KI + VI + NW * 64 - 1) / (NW * 64);  // items per thread
};

// x = h1 + h2 + h3 exactly: three bf16 truncations (8 significant bits
// each) of a float and its remainders; returns the bf16 bit patterns.
__device__ __forceinline__ void split3_bf16(float x, uint32_t& h1, uint32_t& h2, uint32_t& h3) {
  const uint32_t b1 = __float_as_uint(x) & 0xffff0000u;
  const float r1 = x - __uint_as_float(b1);
  const uint32_t b2 = __float_as_uint(r1) & 0xffff0000u;
  const float r2 = r1 - __uint_as_float(b2);
  h1 = b1 >> 16;
  h2 = b2 >> 16;
  h3 = __float_as_uint(r2) >> 16;
}

// position of key r (0..15) of a 16-key group in the V^T tile: the P^T
// operand slot order (quads 1 and 2 swapped)
__device__ __forceinline__ int vt_pos(int key) { return (key & ~15) | ((key & 4) << 1) | ((key & 8) >> 1) | (key & 3); }

template <typename T, int BITS, int D, int GS>
__global__ void __launch_bounds__(512) sdpa_prefill_mfma_kernel(
    const uint16_t* __restrict__ q, const uint32_t* __restrict__ kp, const uint16_t* __restrict__ ksc,
    const uint16_t* __restrict__ kbi, const uint32_t* __restrict__ vp, const uint16_t* __restrict__ vsc,
    const uint16_t* __restrict__ vbi, int Hq, int Hkv, int Lq, Geometry geo, int causal, int window, float scale,
    uint16_t* __restrict__ out) {
  using SH = PrefillShape<D>;
  using CO = CodeOps<T, BITS>;
  constexpr int BN = SH::BN, NW = SH::NW, KP = SH::KP, VP = SH::VP, KI = SH::KI, VI = SH::VI, IPT = SH::IPT;
  constexpr int KW = D * BITS / 32;  // code words per cache row
  constexpr int G = D / GS;
  constexpr int KS = D / 16;         // k-steps of S^T
  constexpr int KPG = GS / 16;       // k-steps per group
  constexpr int DB = D / 32;         // O^T row blocks
  constexpr uint32_t CMASK = (1u << BITS) - 1u;
  // bias MFMA k slots of group g: 6g .. 6g + 5 = key side [b1 b1 b2 b1 b2 b3],
  // query side [X1 X2 X1 X3 X2 X1] (b = b - OFF s; 1..3 its exact bf16 parts)
  constexpr int SPG = 6;
  constexpr int NBM = (G * SPG + 15) / 16;  // bias MFMAs per 32-key block
  constexpr int BPP = 16 * NBM + 8;         // bias row pitch (bf16)
  __shared__ __align__(16) uint16_t kt_lds[2][BN * KP];
  __shared__ __align__(16) uint16_t vt_lds[2][D * VP];
  __shared__ __align__(16) float ks_lds[2][G][BN];           // s per group and key
  __shared__ __align__(16) uint16_t kbias_lds[2][BN * BPP];  // bias operand rows

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 31, lh = lane >> 5;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const int nrep = Hq / Hkv;
  const int64_t valid = row_valid(geo, b);
  const int64_t rowbase = ((int64_t)b * Hkv + kvh) * geo.cap;  // slot 0 of this (b, kvh)

  // ---- this lane's query row --------------------------------------------
  const int r = blockIdx.x * SH::ROWS + wave * 32 + lc;  // (query, head) row
  const int qi = r / nrep, h = r % nrep;
  const bool row_ok = qi < Lq;
  const int64_t pos = valid - Lq + (row_ok ? qi : Lq - 1);  // logical position of the query
  // key range of the workgroup (rows are ordered by query index)
  const int qi_lo = blockIdx.x * SH::ROWS / nrep;
  const int qi_hi = min(Lq - 1, (blockIdx.x * SH::ROWS + SH::ROWS - 1) / nrep);
  int64_t kend = valid, kbeg = 0;
  if (causal) kend = min(kend, valid - Lq + qi_hi + 1);
  if (window > 0) kbeg = max((int64_t)0, valid - Lq + qi_lo - window + 1);
  kbeg = kbeg / BN * BN;
  // this wave's own row range, for the "tile needs no mask" test
  const int wq_lo = min(Lq - 1, (blockIdx.x * SH::ROWS + wave * 32) / nrep);
  const int64_t wpos_lo = valid - Lq + wq_lo;

  // ---- q' = T(q * T(scale)) as the B operand of S^T (in the code operand's
  // slot order) and X_g = sum of q' over group g ------------------------------
  const float scale_t = Conv<T>::round(scale);
  const bool apply_scale = scale != 1.0f;
  u32x4_t qop[KS];
  float xg[G];
#pragma unroll
  for (int g = 0; g < G; g++) xg[g] = 0.f;
  {
    const uint16_t* qrow = q + (((int64_t)b * Hq + (int64_t)kvh * nrep + h) * Lq + (row_ok ? qi : 0)) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      u32x4_t raw = row_ok ? *reinterpret_cast<const u32x4_t*>(qrow + 16 * ks + 8 * lh) : u32x4_t{0u, 0u, 0u, 0u};
      if (apply_scale) {
#pragma unroll
        for (int p2 = 0; p2 < 4; p2++) {
          const float lo = Conv<T>::round(Conv<T>::from_bits(raw[p2] & 0xffffu) * scale_t);
          const float hi = Conv<T>::round(Conv<T>::from_bits(raw[p2] >> 16) * scale_t);
          raw[p2] = Mma<T>::pack2(lo, hi);
        }
      }
      float part = 0.f;
#pragma unroll
      for (int p2 = 0; p2 < 4; p2++)
        part += Conv<T>::from_bits(raw[p2] & 0xffffu) + Conv<T>::from_bits(raw[p2] >> 16);
      xg[ks / KPG] += part;
      qop[ks] = permute8<CO::ORDER>(raw);
    }
  }
#pragma unroll
  for (int g = 0; g < G; g++) xg[g] += __shfl_xor(xg[g], 32);
  // B operand of the bias MFMAs: slot sg = 16 m + 8 lh + e
  u32x4_t xop[NBM];
  {
    uint32_t xs[G][3];
#pragma unroll
    for (int g = 0; g < G; g++) split3_bf16(xg[g], xs[g][0], xs[g][1], xs[g][2]);
    constexpr int PART[SPG] = {0, 1, 0, 2, 1, 0};
    auto slot = [&](int sg) -> uint32_t { return sg < G * SPG ? xs[sg / SPG][PART[sg % SPG]] : 0u; };
#pragma unroll
    for (int m = 0; m < NBM; m++)
#pragma unroll
      for (int p2 = 0; p2 < 4; p2++) {
        const int s0 = 16 * m + 2 * p2;
        const uint32_t w0 = slot(s0) | (slot(s0 + 1) << 16), w1 = slot(s0 + 8) | (slot(s0 + 9) << 16);
        xop[m][p2] = lh ? w1 : w0;
      }
  }
  // key-side pad slots G * SPG .. 16 NBM stay zero (staging never writes them)
  if constexpr (G * SPG < 16 * NBM) {
    for (int i = tid; i < 2 * BN * (16 * NBM - G * SPG); i += NW * 64) {
      const int per = 16 * NBM - G * SPG, row = i / per;
      kbias_lds[row / BN][(row % BN) * BPP + G * SPG + i % per] = 0;
    }
  }

  // ---- K/V tile loads: item it < KI is (key it / (D/32), 32 codes), else
  // (4 keys, 8 codes) of V with the key quad fastest across lanes (the V^T
  // writes of one instruction then land on distinct LDS banks); loads are
  // raw buffer loads bounded to the row's valid keys (keys past them read 0)
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp + rowbase * KW, (uint32_t)(valid * KW * 4));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp + rowbase * KW, (uint32_t)(valid * KW * 4));
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksc + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rkb = make_rsrc(kbi + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(vsc + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rvb = make_rsrc(vbi + rowbase * G, (uint32_t)(valid * G * 2));
  constexpr int KIW = 32 * BITS / 32;  // words per K item (4 or 8)
  constexpr int VIW = 8 * BITS / 32;   // words per key of a V item (1 or 2)
  uint32_t reg_w[IPT][8];
  uint32_t reg_s[IPT][4], reg_b[IPT][4];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int u = 0; u < IPT; u++) {
      const int it = tid + u * NW * 64;
      if (it < KI) {
        const int key = it / (D / 32), qd = it % (D / 32);
        const uint32_t roff = (uint32_t)(k0 + key) * (uint32_t)(KW * 4) + (uint32_t)qd * KIW * 4;
        const u32x4_t w0 = buf_load128(rk, roff, 0u);
        reg_w[u][0] = w0.x; reg_w[u][1] = w0.y; reg_w[u][2] = w0.z; reg_w[u][3] = w0.w;
        if constexpr (KIW == 8) {
          const u32x4_t w1 = buf_load128(rk, roff + 16u, 0u);
          reg_w[u][4] = w1.x; reg_w[u][5] = w1.y; reg_w[u][6] = w1.z; reg_w[u][7] = w1.w;
        }
        const uint32_t so = ((uint32_t)(k0 + key) * G + (uint32_t)(32 * qd / GS)) * 2u;
        reg_s[u][0] = buf_load16(rks, so, 0u);
        reg_b[u][0] = buf_load16(rkb, so, 0u);
      } else if (it < KI + VI) {
        const int vi = it - KI, kq = vi % (BN / 4), d8 = vi / (BN / 4);
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          const uint32_t roff = (uint32_t)(k0 + 4 * kq + kk) * (uint32_t)(KW * 4) + (uint32_t)d8 * VIW * 4;
          if constexpr (VIW == 1) {
            reg_w[u][kk] = buf_load32(rv, roff, 0u);
          } else {
            const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(rv, (int)roff, 0, 0);
            reg_w[u][2 * kk] = v2[0];
            reg_w[u][2 * kk + 1] = v2[1];
          }
          const uint32_t so = ((uint32_t)(k0 + 4 * kq + kk) * G + (uint32_t)(8 * d8 / GS)) * 2u;
          reg_s[u][kk] = buf_load16(rvs, so, 0u);
          reg_b[u][kk] = buf_load16(rvb, so, 0u);
        }
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int u = 0; u < IPT; u++) {
      const int it = tid + u * NW * 64;
      if (it < KI) {
        const int key = it / (D / 32), qd = it % (D / 32);
        uint16_t* dst = &kt_lds[buf][key * KP + 32 * qd];
#pragma unroll
        for (int j = 0; j < 4; j++) {  // 8 codes -> 8 exact operands (OFF + c)
          if constexpr (BITS == 4)
            *reinterpret_cast<u32x4_t*>(dst + 8 * j) = CO::operand(reg_w[u][j]);
          else
            *reinterpret_cast<u32x4_t*>(dst + 8 * j) = CO::operand(reg_w[u][2 * j], reg_w[u][2 * j + 1]);
        }
        if ((32 * qd) % GS == 0) {  // the group's first item writes its s and bias slots
          const float sc = Conv<T>::from_bits(reg_s[u][0]), bi = Conv<T>::from_bits(reg_b[u][0]);
          const int g = 32 * qd / GS;
          ks_lds[buf][g][key] = sc;
          uint32_t h1, h2, h3;
          split3_bf16(__builtin_fmaf(-CO::OFFSET, sc, bi), h1, h2, h3);
          uint32_t* brow = reinterpret_cast<uint32_t*>(&kbias_lds[buf][key * BPP + SPG * g]);
          brow[0] = h1 | (h1 << 16);
          brow[1] = h2 | (h1 << 16);
          brow[2] = h2 | (h3 << 16);
        }
      } else if (it < KI + VI) {
        const int vi = it - KI, kq = vi % (BN / 4), d8 = vi / (BN / 4);
        float sc[4], bi[4];
#pragma unroll
        for (int kk = 0; kk < 4; kk++) {
          sc[kk] = Conv<T>::from_bits(reg_s[u][kk]);
          bi[kk] = Conv<T>::from_bits(reg_b[u][kk]);
        }
        const int p0 = vt_pos(4 * kq);  // the 4 keys stay adjacent
#pragma unroll
        for (int e = 0; e < 8; e++) {  // d = 8 d8 + e
          float v[4];
#pragma unroll
          for (int kk = 0; kk < 4; kk++) {
            const uint32_t wv = reg_w[u][kk * VIW + e * BITS / 32];
            v[kk] = __builtin_fmaf(sc[kk], (float)((wv >> ((e * BITS) % 32)) & CMASK), bi[kk]);
          }
          *reinterpret_cast<uint2*>(&vt_lds[buf][(8 * d8 + e) * VP + p0]) =
              make_uint2(Mma<T>::pack2(v[0], v[1]), Mma<T>::pack2(v[2], v[3]));
        }
      }
    }
  };

  f32x16_t oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; i++)
#pragma unroll
    for (int e = 0; e < 16; e++) oacc[i][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // Tile t's K/V sit in LDS buffer t & 1; tile t + 1's codes arrive in
  // registers during tile t - 1 and are staged into the other buffer during
  // tile t (that buffer's readers passed the previous barrier).  The two
  // waves sharing a SIMD (w and w + NW/2) take the score MFMAs and the
  // staging VALU in opposite orders, so one uses the matrix core while the
  // other dequantizes.  (Alternating the softmax / P V phases as well needs
  // both orders' live ranges at once and spills.)
  if (kbeg < kend) {
    load(kbeg);
    stash(0);
    if (kbeg + BN < kend) load(kbeg + BN);
  }
  lds_barrier();
  const bool mfma_first = wave < NW / 2;
  int buf = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += BN) {
    const bool more = k0 + BN < kend;
    // ---- S^T: two 32-key blocks, one group at a time ------------------------
    // key of sacc[kb][v]: 32 kb + 8 (v / 4) + 4 lh + v % 4 (four consecutive
    // keys per v / 4, whose (s, b - OFF s) are one 16-byte LDS read each)
    f32x16_t sacc[2];
    auto scores = [&]() {
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        f32x16_t acc;
#pragma unroll
        for (int e = 0; e < 16; e++) acc[e] = 0.f;
#pragma unroll
        for (int m = 0; m < NBM; m++) {
          const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&kbias_lds[buf][(32 * kb + lc) * BPP + 16 * m + 8 * lh]);
          acc = mma32<BF16>(a, xop[m], acc);
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
          // chained MFMAs on one accumulator forward C, so a block's groups
          // run back to back; only one 16-register partial is live
          f32x16_t part;
#pragma unroll
          for (int e = 0; e < 16; e++) part[e] = 0.f;
#pragma unroll
          for (int kk = 0; kk < KPG; kk++) {
            const int ks = g * KPG + kk;
            const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&kt_lds[buf][(32 * kb + lc) * KP + 16 * ks + 8 * lh]);
            part = mma32<T>(a, qop[ks], part);
          }
#pragma unroll
          for (int r4 = 0; r4 < 4; r4++) {
            const float4 sv = *reinterpret_cast<const float4*>(&ks_lds[buf][g][32 * kb + 8 * r4 + 4 * lh]);
            acc[4 * r4 + 0] = __builtin_fmaf(sv.x, part[4 * r4 + 0], acc[4 * r4 + 0]);
            acc[4 * r4 + 1] = __builtin_fmaf(sv.y, part[4 * r4 + 1], acc[4 * r4 + 1]);
            acc[4 * r4 + 2] = __builtin_fmaf(sv.z, part[4 * r4 + 2], acc[4 * r4 + 2]);
            acc[4 * r4 + 3] = __builtin_fmaf(sv.w, part[4 * r4 + 3], acc[4 * r4 + 3]);
          }
        }
        sacc[kb] = acc;
      }
      // the scores are final here: keeps the fold from being merged with the
      // other order's copy below the staging (its partials would stay live)
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int v = 0; v < 16; v++) asm volatile("" : "+v"(sacc[kb][v]));
    };
    if (mfma_first) {
      scores();
      if (more) stash(buf ^ 1);
    } else {
      if (more) stash(buf ^ 1);
      scores();
    }
    if (k0 + 2 * BN < kend) load(k0 + 2 * BN);
    // ---- online softmax over this lane's 32 keys (+ lane ^ 32's) -----------
    // key of sacc[kb][v]: k0 + 32 kb + 8 (v / 4) + 4 lh + v % 4
    const bool need_mask = k0 + BN > valid || (causal && k0 + BN - 1 > wpos_lo) ||
                           (window > 0 && k0 <= valid - Lq + min(Lq - 1, wq_lo + 32) - window);
    // scores stay in natural units (the running max too); log2(e) enters
    // each exponent through one fma
    float tmax = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        float sv = sacc[kb][v];
        if (need_mask) {  // wave-uniform
          const int64_t j = k0 + 32 * kb + 8 * (v / 4) + 4 * lh + v % 4;
          const bool ok = j < valid && (!causal || j <= pos) && (window <= 0 || pos < j + window) && row_ok;
          sv = ok ? sv : -INFINITY;
        }
        sacc[kb][v] = sv;
        tmax = fmaxf(tmax, sv);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_old = m_run;
    const float m_new = tmax > m_old + 8.0f / LOG2E ? tmax : m_old;  // lazy: p <= 2^8
    const float alpha = m_new == m_old ? 1.0f : __builtin_amdgcn_exp2f((m_old - m_new) * LOG2E);
    const float m_sub = m_new == -INFINITY ? 0.0f : -m_new * LOG2E;
    m_run = m_new;
    float psum[4] = {0.f, 0.f, 0.f, 0.f};  // four chains: the sum of exactly the P the MFMA sees
    uint32_t pk[2][8];  // P as T pairs: [block][pair]
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][v], LOG2E, m_sub));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kb][v + 1], LOG2E, m_sub));
        pk[kb][v / 2] = Mma<T>::pack2(p0, p1);
        psum[(v / 2) % 4] = Mma<T>::sum2(pk[kb][v / 2], psum[(v / 2) % 4]);
      }
    l_run = l_run * alpha + ((psum[0] + psum[1]) + (psum[2] + psum[3]));
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < DB; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) oacc[i][e] *= alpha;
    }
    // ---- O^T += V^T P^T: four 16-key k-steps --------------------------------
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const int kb = m / 2, vo = 4 * (m % 2);
      const u32x4_t bop = {pk[kb][vo], pk[kb][vo + 1], pk[kb][vo + 2], pk[kb][vo + 3]};
#pragma unroll
      for (int i = 0; i < DB; i++) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(&vt_lds[buf][(32 * i + lc) * VP + 16 * m + 8 * lh]);
        oacc[i] = mma32<T>(a, bop, oacc[i]);
      }
    }
    lds_barrier();
    buf ^= 1;
  }

  // ---- normalise and store: lane holds d = 32 i + 8 (v / 4) + 4 lh + v % 4 --
  const float lt = l_run + __shfl_xor(l_run, 32);
  const float inv = lt > 0.f ? 1.0f / lt : 0.f;
  if (row_ok) {
    uint16_t* orow = out + (((int64_t)b * Hq + (int64_t)kvh * nrep + h) * Lq + qi) * D;
#pragma unroll
    for (int i = 0; i < DB; i++)
#pragma unroll
      for (int v = 0; v < 16; v += 4) {
        const int d = 32 * i + 8 * (v / 4) + 4 * lh;
        *reinterpret_cast<uint2*>(orow + d) = make_uint2(Mma<T>::pack2(oacc[i][v] * inv, oacc[i][v + 1] * inv),
                                                         Mma<T>::pack2(oacc[i][v + 2] * inv, oacc[i][v + 3] * inv));
      }
  }
}

// ===================================================== MFMA prefill, wide rows
//
// Lq > 1 at head_dim 256 / 512 (Gemma4's full-attention layers, the only
// ones with a quantized cache): the kernel above keeps a 32-row block's whole
// output (D/32 accumulator tiles) and q' (D/16 operands) in registers, which
// does not fit past D = 128.  Here a wave owns 16 (query, head) rows as the
// rows of v_mfma_f32_16x16x32 (4 waves, one per SIMD: its D/16 accumulator
// tiles and q' operands take most of a SIMD's registers).
// Per 32-key tile, shared by the workgroup through a double-buffered LDS:
//   * K as exact code operands OFF + c plus fp32 per-key (s, b - OFF s); the
//     scores S = s (C q'^T) + (b - OFF s) X per group (lane quarter lq holds
//     codes [lq gs/4, (lq+1) gs/4) of each group), no rounding of K;
//   * V dequantized (fp32 s * c + b -> T) and transposed;
//   * online softmax per row (natural units, log2(e) in each exponent),
//     causal / window masks on boundary tiles only;
//   * P goes through the wave's own LDS rows into the A operand of O += P V
//     (no barrier: a wave's LDS accesses stay in order).
template <int D, int GS, int BITS>
struct PrefillWideShape {
  static constexpr int NW = 4;                    // waves (16 rows each), one per SIMD
  static constexpr int ROWS = 16 * NW;
  static constexpr int NT = NW * 64;
  static constexpr int TK = 32;                   // keys per tile
  static constexpr int G = D / GS;
  static constexpr int KW = D * BITS / 32;        // code words per cache row
  static constexpr int CPQ = GS / 4, KST = GS / 32;
  static constexpr int KP = D + 8;                // K tile pitch (T)
  static constexpr int VP = TK + 8;               // V^T / P pitch (T)
  static constexpr int UW = BITS / 4;             // code words per 8-code unit
  static constexpr int KIT = TK * D / 8 / NT;     // K units (8 codes) per thread per tile
  static constexpr int VI = (TK / 8) * (D / 8);   // V items: 8 keys x 8 dims
  static constexpr int SI = TK * G;               // K (s, b) items
  static constexpr int DC = D / 16;               // output column tiles
};

template <typename T, int BITS, int D, int GS>
__global__ void __launch_bounds__(256) sdpa_prefill_wide_kernel(
    const uint16_t* __restrict__ q, const uint32_t* __restrict__ kp, const uint16_t* __restrict__ ksc,
    const uint16_t* __restrict__ kbi, const uint32_t* __restrict__ vp, const uint16_t* __restrict__ vsc,
    const uint16_t* __restrict__ vbi, int Hq, int Hkv, int Lq, Geometry geo, int causal, int window, float scale,
    uint16_t* __restrict__ out, int nsplit, float* __restrict__ part_o, float2* __restrict__ part_ml) {
  using SH = PrefillWideShape<D, GS, BITS>;
  using CO = CodeOps<T, BITS>;
  constexpr int NW = SH::NW, ROWS = SH::ROWS, NT = SH::NT, TK = SH::TK, G = SH::G, KW = SH::KW, CPQ = SH::CPQ;
  constexpr int KST = SH::KST, KP = SH::KP, VP = SH::VP, UW = SH::UW, KIT = SH::KIT, VI = SH::VI, SI = SH::SI;
  constexpr int DC = SH::DC;
  constexpr float OFF = CO::OFFSET;
  constexpr uint32_t CMASK = (1u << BITS) - 1u;
  static_assert(KIT >= 1 && VI <= NT && SI <= NT && G <= 8 && NT == 256, "wide prefill geometry");
  __shared__ __align__(16) uint16_t kt_lds[2][TK * KP];
  __shared__ __align__(16) uint16_t vt_lds[2][D * VP];
  __shared__ __align__(16) float ksb[2][2][G][TK];  // [buf][s | b - OFF s][group][key]
  __shared__ __align__(16) uint16_t pw[NW][16 * VP];  // each wave's P rows
  __shared__ __align__(16) float xw[NW][G][16];       // each wave's X[group][row]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ln = lane & 15, lq = lane >> 4;
  const int b = blockIdx.z, kvh = blockIdx.y;
  const int nrep = Hq / Hkv;
  const int64_t valid = row_valid(geo, b);
  const int64_t rowbase = ((int64_t)b * Hkv + kvh) * geo.cap;

  // ---- rows: r = query * nrep + head; the A operand's row is ln, the
  // accumulator rows are 4 lq + i.  blockIdx.x = row block * nsplit + key
  // split ---------------------------------------------------------------------
  const int rb = (int)blockIdx.x / nsplit, sp = (int)blockIdx.x % nsplit;
  const int r0 = rb * ROWS + 16 * wave;
  int64_t pos[4];
  bool rok[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = r0 + 4 * lq + i, qi = r / nrep;
    rok[i] = qi < Lq;
    pos[i] = valid - Lq + (rok[i] ? qi : Lq - 1);
  }
  const int qi_lo = rb * ROWS / nrep;
  const int qi_hi = min(Lq - 1, (rb * ROWS + ROWS - 1) / nrep);
  int64_t kend = valid, kbeg = 0;
  if (causal) kend = min(kend, valid - Lq + qi_hi + 1);
  if (window > 0) kbeg = max((int64_t)0, valid - Lq + qi_lo - window + 1);
  kbeg = kbeg / TK * TK;
  if (nsplit > 1) {  // this split's whole tiles of the row block's key range (maybe none)
    const int64_t ntk = kend > kbeg ? (kend - kbeg + TK - 1) / TK : 0;
    const int64_t per = (ntk + nsplit - 1) / nsplit;
    const int64_t s0 = kbeg + (int64_t)sp * per * TK;
    kend = min(kend, s0 + per * TK);
    kbeg = s0;
  }
  const int wq_lo = min(Lq - 1, r0 / nrep), wq_hi = min(Lq - 1, (r0 + 15) / nrep);
  const int64_t wpos_lo = valid - Lq + wq_lo, wpos_hi = valid - Lq + wq_hi;

  // ---- q' operand (row ln, quarter lq) and X[group][row] -------------------
  const float scale_t = Conv<T>::round(scale);
  const bool apply_scale = scale != 1.0f;
  u32x4_t qop[G][KST];
  {
    const int ra = r0 + ln, qa = ra / nrep, ha = ra % nrep;
    const bool aok = qa < Lq;
    const uint16_t* qrow = q + (((int64_t)b * Hq + (int64_t)kvh * nrep + ha) * Lq + (aok ? qa : 0)) * D;
#pragma unroll
    for (int g = 0; g < G; g++) {
      float xp = 0.f;
#pragma unroll
      for (int s = 0; s < KST; s++) {
        u32x4_t raw = aok ? *reinterpret_cast<const u32x4_t*>(qrow + g * GS + lq * CPQ + 8 * s) : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int p2 = 0; p2 < 4; p2++) {
          const float lo = scaled_q<T>(Conv<T>::from_bits(raw[p2] & 0xffffu), scale_t, apply_scale);
          const float hi = scaled_q<T>(Conv<T>::from_bits(raw[p2] >> 16), scale_t, apply_scale);
          raw[p2] = Mma<T>::pack2(lo, hi);
          xp += lo + hi;
        }
        qop[g][s] = permute8<CO::ORDER>(raw);
      }
      xp += __shfl_xor(xp, 16);
      xp += __shfl_xor(xp, 32);
      if (lq == 0) xw[wave][g][ln] = xp;
    }
  }

  // ---- K/V tile staging (raw buffer loads bounded to the valid keys) --------
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp + rowbase * KW, (uint32_t)(valid * KW * 4));
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp + rowbase * KW, (uint32_t)(valid * KW * 4));
  const __amdgpu_buffer_rsrc_t rks = make_rsrc(ksc + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rkb = make_rsrc(kbi + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rvs = make_rsrc(vsc + rowbase * G, (uint32_t)(valid * G * 2));
  const __amdgpu_buffer_rsrc_t rvb = make_rsrc(vbi + rowbase * G, (uint32_t)(valid * G * 2));
  constexpr uint32_t OOB = 0x80000000u;
  const bool sact = tid < SI, vact = tid < VI;
  const int s_key = tid / G, s_g = tid % G;      // K (s, b) item
  const int v_ko = tid % (TK / 8), v_vd = tid / (TK / 8);  // V item: key octet, 8-dim block
  const int v_g = 8 * v_vd / GS;
  uint32_t kw[KIT][UW];
  uint32_t ksr, kbr;
  uint32_t vw[8][UW], vsr[8], vbr[8];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int it = 0; it < KIT; it++) {
      const int u = tid + NT * it, key = u / (D / 8), c8 = u % (D / 8);
      const uint32_t off = ((uint32_t)(k0 + key) * KW + (uint32_t)c8 * UW) * 4u;
      if constexpr (UW == 1) {
        kw[it][0] = buf_load32(rk, off, 0u);
      } else {
        const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(rk, (int)off, 0, 0);
        kw[it][0] = v2[0];
        kw[it][1] = v2[1];
      }
    }
    const uint32_t so = sact ? (((uint32_t)(k0 + s_key) * G + (uint32_t)s_g) * 2u) & ~3u : OOB;
    ksr = __builtin_amdgcn_raw_buffer_load_b32(rks, (int)so, 0, 0);
    kbr = __builtin_amdgcn_raw_buffer_load_b32(rkb, (int)so, 0, 0);
#pragma unroll
    for (int kk = 0; kk < 8; kk++) {
      const uint32_t key = (uint32_t)(k0 + 8 * v_ko + kk);
      const uint32_t off = vact ? (key * KW + (uint32_t)v_vd * UW) * 4u : OOB;
      if constexpr (UW == 1) {
        vw[kk][0] = buf_load32(rv, off, 0u);
      } else {
        const auto v2 = __builtin_amdgcn_raw_buffer_load_b64(rv, (int)off, 0, 0);
        vw[kk][0] = v2[0];
        vw[kk][1] = v2[1];
      }
      const uint32_t vso = vact ? ((key * (uint32_t)G + (uint32_t)v_g) * 2u) & ~3u : OOB;
      vsr[kk] = __builtin_amdgcn_raw_buffer_load_b32(rvs, (int)vso, 0, 0);
      vbr[kk] = __builtin_amdgcn_raw_buffer_load_b32(rvb, (int)vso, 0, 0);
    }
  };
  auto stash = [&](int64_t k0, int buf) {
#pragma unroll
    for (int it = 0; it < KIT; it++) {
      const int u = tid + NT * it, key = u / (D / 8), c8 = u % (D / 8);
      u32x4_t op;
      if constexpr (BITS == 4)
        op = CO::operand(kw[it][0]);
      else
        op = CO::operand(kw[it][0], kw[it][1]);
      *reinterpret_cast<u32x4_t*>(&kt_lds[buf][key * KP + 8 * c8]) = op;
    }
    if (sact) {
      const int sh = 16 * (int)((((uint32_t)(k0 + s_key) * G + (uint32_t)s_g)) & 1u);
      const float sc = Conv<T>::from_bits((ksr >> sh) & 0xffffu), bi = Conv<T>::from_bits((kbr >> sh) & 0xffffu);
      ksb[buf][0][s_g][s_key] = sc;
      ksb[buf][1][s_g][s_key] = __builtin_fmaf(-OFF, sc, bi);
    }
    if (vact) {
      float sc[8], bi[8];
#pragma unroll
      for (int kk = 0; kk < 8; kk++) {
        const int sh = 16 * (int)((((uint32_t)(k0 + 8 * v_ko + kk) * G + (uint32_t)v_g)) & 1u);
        sc[kk] = Conv<T>::from_bits((vsr[kk] >> sh) & 0xffffu);
        bi[kk] = Conv<T>::from_bits((vbr[kk] >> sh) & 0xffffu);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float x[8];
#pragma unroll
        for (int kk = 0; kk < 8; kk++) {
          const uint32_t wv = vw[kk][e * BITS / 32];
          x[kk] = __builtin_fmaf(sc[kk], (float)((wv >> ((e * BITS) % 32)) & CMASK), bi[kk]);
        }
        *reinterpret_cast<u32x4_t*>(&vt_lds[buf][(8 * v_vd + e) * VP + 8 * v_ko]) =
            u32x4_t{Mma<T>::pack2(x[0], x[1]), Mma<T>::pack2(x[2], x[3]), Mma<T>::pack2(x[4], x[5]),
                    Mma<T>::pack2(x[6], x[7])};
      }
    }
  };

  f32x4_t oacc[DC];
#pragma unroll
  for (int c = 0; c < DC; c++) oacc[c] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float m_run[4], l_run[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m_run[i] = -INFINITY;
    l_run[i] = 0.f;
  }

  if (kbeg < kend) {
    load(kbeg);
    stash(kbeg, 0);
    if (kbeg + TK < kend) load(kbeg + TK);
  }
  lds_barrier();
  int buf = 0;
  for (int64_t k0 = kbeg; k0 < kend; k0 += TK) {
    // ---- scores: two 16-key column tiles, one group at a time -------------
    f32x4_t sacc[2];
#pragma unroll
    for (int ct = 0; ct < 2; ct++) {
      sacc[ct] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < G; g++) {
        f32x4_t part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KST; s++) {
          const u32x4_t bop =
              *reinterpret_cast<const u32x4_t*>(&kt_lds[buf][(16 * ct + ln) * KP + g * GS + lq * CPQ + 8 * s]);
          part = Mma<T>::mma(qop[g][s], bop, part);
        }
        const float sk = ksb[buf][0][g][16 * ct + ln], bk = ksb[buf][1][g][16 * ct + ln];
        const float4 xv = *reinterpret_cast<const float4*>(&xw[wave][g][4 * lq]);
        const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
        for (int i = 0; i < 4; i++) sacc[ct][i] = __builtin_fmaf(sk, part[i], __builtin_fmaf(bk, xa[i], sacc[ct][i]));
      }
    }
    if (k0 + TK < kend) stash(k0 + TK, buf ^ 1);
    if (k0 + 2 * TK < kend) load(k0 + 2 * TK);
    // ---- online softmax over this tile's 32 keys ---------------------------
    const bool need_mask = k0 + TK > valid || (causal && k0 + TK - 1 > wpos_lo) ||
                           (window > 0 && k0 <= wpos_hi - window);
    float alpha[4], msub[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int ct = 0; ct < 2; ct++) {
        if (need_mask) {  // wave-uniform
          const int64_t j = k0 + 16 * ct + ln;
          const bool ok = j < valid && (!causal || j <= pos[i]) && (window <= 0 || pos[i] < j + window) && rok[i];
          sacc[ct][i] = ok ? sacc[ct][i] : -INFINITY;
        }
      }
      float mv = fmaxf(sacc[0][i], sacc[1][i]);
      mv = fmaxf(mv, __shfl_xor(mv, 1));
      mv = fmaxf(mv, __shfl_xor(mv, 2));
      mv = fmaxf(mv, __shfl_xor(mv, 4));
      mv = fmaxf(mv, __shfl_xor(mv, 8));
      const float m_old = m_run[i];
      const float m_new = mv > m_old + 8.0f / LOG2E ? mv : m_old;  // lazy: p <= 2^8
      alpha[i] = m_new == m_old ? 1.0f : __builtin_amdgcn_exp2f((m_old - m_new) * LOG2E);
      msub[i] = m_new == -INFINITY ? 0.0f : -m_new * LOG2E;
      m_run[i] = m_new;
    }
    float psum[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      psum[i] = 0.f;
#pragma unroll
      for (int ct = 0; ct < 2; ct++) {
        const uint32_t pb = Conv<T>::to_bits(__builtin_amdgcn_exp2f(__builtin_fmaf(sacc[ct][i], LOG2E, msub[i])));
        pw[wave][(4 * lq + i) * VP + 16 * ct + ln] = (uint16_t)pb;
        psum[i] += Conv<T>::from_bits(pb);  // the P the MFMA sees
      }
      l_run[i] = l_run[i] * alpha[i] + psum[i];
    }
    if (__any(alpha[0] != 1.0f || alpha[1] != 1.0f || alpha[2] != 1.0f || alpha[3] != 1.0f)) {
#pragma unroll
      for (int c = 0; c < DC; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) oacc[c][i] *= alpha[i];
    }
    // ---- O += P V: one 32-key k-step per 16-dim column tile ---------------
    const u32x4_t pa = *reinterpret_cast<const u32x4_t*>(&pw[wave][ln * VP + 8 * lq]);
#pragma unroll
    for (int c = 0; c < DC; c++) {
      const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(&vt_lds[buf][(16 * c + ln) * VP + 8 * lq]);
      oacc[c] = Mma<T>::mma(pa, bv, oacc[c]);
    }
    lds_barrier();
    buf ^= 1;
  }

  // ---- normalise and store: lane holds dims 16 c + ln of rows 4 lq + i ---
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float lv = l_run[i];
    lv += __shfl_xor(lv, 1);
    lv += __shfl_xor(lv, 2);
    lv += __shfl_xor(lv, 4);
    lv += __shfl_xor(lv, 8);
    const float inv = lv > 0.f ? 1.0f / lv : 0.f;
    if (rok[i]) {
      const int r = r0 + 4 * lq + i, qd = r / nrep, hd = r % nrep;
      if (nsplit == 1) {
        uint16_t* orow = out + (((int64_t)b * Hq + (int64_t)kvh * nrep + hd) * Lq + qd) * D;
#pragma unroll
        for (int c = 0; c < DC; c++) orow[16 * c + ln] = (uint16_t)Conv<T>::to_bits(oacc[c][i] * inv);
      } else {  // (U, M in log2 units, L) of row (hd, qd) for the merge kernel
        const int64_t prow = (((int64_t)b * Hkv + kvh) * nsplit + sp) * ((int64_t)nrep * Lq) + (int64_t)hd * Lq + qd;
#pragma unroll
        for (int c = 0; c < DC; c++) part_o[prow * D + 16 * c + ln] = oacc[c][i];
        if (ln == 0) part_ml[prow] = make_float2(m_run[i] * LOG2E, lv);
      }
    }
  }
}

template <typename T, int BITS>
int launch_prefill_wide(int D, int gs, const void* q, int B, int Hq, int Hkv, int Lq, const uint32_t* kp,
                        const void* ks, const void* kb, const uint32_t* vp, const void* vs, const void* vb,
                        Geometry geo, int causal, int window, float scale, void* out, hipStream_t s,
                        const mlxq::Scratch& scr) {
  const int nrep = Hq / Hkv;
  const int64_t rows = (int64_t)Lq * nrep;
  // Fewer row blocks than CUs (one 4-wave workgroup fills a CU): split each
  // row block's keys over nsplit workgroups, at least 8 tiles of 32 keys
  // each, and merge their partials with the decode merge kernel.
  const int64_t span = geo.valid_len ? geo.cap : geo.n_kv;
  const int64_t wgs = (rows + 63) / 64 * Hkv * B;
  const int64_t cus = mlxq::device_cu_count();
  int nsplit = 1;
  if (wgs < cus && rows * D < ((int64_t)1 << 31)) {
    const int64_t by_cus = (cus + wgs - 1) / wgs, by_keys = span / (8 * 32);
    nsplit = (int)std::max<int64_t>(1, std::min<int64_t>(std::min(by_cus, by_keys), 16));
  }
  float* part_o = nullptr;
  float2* part_ml = nullptr;
  if (nsplit > 1) {
    const size_t slots = (size_t)B * Hkv * nsplit;
    const size_t obytes = (slots * rows * D * sizeof(float) + 255) & ~(size_t)255;
    void* pws = nullptr;
    int rc = scr.get(obytes + slots * rows * sizeof(float2), &pws, s);
    if (rc) return rc;
    part_o = (float*)pws;
    part_ml = (float2*)((uint8_t*)pws + obytes);
  }
#define PREW(DV, GV)                                                                                           \
  if (D == DV && gs == GV) {                                                                                   \
    using SH = PrefillWideShape<DV, GV, BITS>;                                                                 \
    static_assert(SH::ROWS == 64 && SH::TK == 32, "split sizing above");                                       \
    dim3 grid((unsigned)((rows + SH::ROWS - 1) / SH::ROWS * nsplit), (unsigned)Hkv, (unsigned)B);              \
    hipLaunchKernelGGL((sdpa_prefill_wide_kernel<T, BITS, DV, GV>), grid, dim3(SH::NT), 0, s,                  \
                       (const uint16_t*)q, kp, (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs, \
                       (const uint16_t*)vb, Hq, Hkv, Lq, geo, causal, window, scale, (uint16_t*)out, nsplit,   \
                       part_o, part_ml);                                                                       \
    MLXQ_LAUNCHED("sdpa_prefill_wide_kernel");                                                                 \
    if (nsplit > 1) {                                                                                          \
      const int64_t cols = rows * D / 4;                                                                       \
      dim3 mgrid((unsigned)((cols + 63) / 64), (unsigned)Hkv, (unsigned)B);                                    \
      const int mrc = launch_merge<T>(mgrid, nsplit, s, part_o, part_ml, (int)(Hq * (int64_t)Lq), Hkv, D, geo, \
                                      0, (uint16_t*)out);                                                      \
      if (mrc) return mrc;                                                                                     \
    }                                                                                                          \
    return MLXQ_OK;                                                                                            \
  }
  PREW(256, 32) PREW(256, 64) PREW(256, 128) PREW(512, 64) PREW(512, 128)
#undef PREW
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "prefill: no wide MFMA instance for this head_dim/group_size");
}

template <typename T, int BITS>
int launch_prefill(int D, int gs, const void* q, int B, int Hq, int Hkv, int Lq, const uint32_t* kp, const void* ks,
                   const void* kb, const uint32_t* vp, const void* vs, const void* vb, Geometry geo, int causal,
                   int window, float scale, void* out, hipStream_t s) {
  const int nrep = Hq / Hkv;
  const int64_t rows = (int64_t)Lq * nrep;
#define PRE(DV, GV)                                                                                            \
  if (D == DV && gs == GV) {                                                                                   \
    dim3 grid((unsigned)((rows + PrefillShape<DV>::ROWS - 1) / PrefillShape<DV>::ROWS), (unsigned)Hkv, (unsigned)B); \
    hipLaunchKernelGGL((sdpa_prefill_mfma_kernel<T, BITS, DV, GV>), grid, dim3(512), 0, s, (const uint16_t*)q, kp, \
                       (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs, (const uint16_t*)vb, Hq, Hkv, \
                       Lq, geo, causal, window, scale, (uint16_t*)out);                                        \
    MLXQ_LAUNCHED("sdpa_prefill_mfma_kernel");                                                                 \
    return MLXQ_OK;                                                                                            \
  }
  PRE(64, 32) PRE(64, 64) PRE(128, 32) PRE(128, 64) PRE(128, 128)
#undef PRE
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "prefill: no MFMA instance for this head_dim/group_size");
}

// ========================================================== generic kernel
// One workgroup (128 threads) per (batch row, q head, query).  Scores for
// 128 keys at a time (one key per thread, fp32 dot of fp32-dequantized K),
// online softmax through LDS, values accumulated with threads over d.
// With an array mask (amask != null; causal = window = 0) key j of query i
// of row b is attended iff amask[b mask_bs + i mask_rs + j] != 0, and a
// query with no attended key averages V over all its valid keys: the
// reference's where(mask, scores, FINFO_MIN) followed by a softmax gives
// every key the same weight when all of them are masked.
template <typename T, int BITS>
__global__ void __launch_bounds__(128) sdpa_generic_kernel(
    const void* __restrict__ qv, const uint32_t* __restrict__ kp, const void* __restrict__ ksv,
    const void* __restrict__ kbv, const uint32_t* __restrict__ vp, const void* __restrict__ vsv,
    const void* __restrict__ vbv, int Hq, int Hkv, int Lq, int D, int gs, Geometry geo, int causal, int window,
    float scale, void* __restrict__ outv, const uint8_t* __restrict__ amask = nullptr, int64_t mask_bs = 0,
    int64_t mask_rs = 0) {
  using S = typename T::storage;
  const S* q = reinterpret_cast<const S*>(qv);
  const S* ks = reinterpret_cast<const S*>(ksv);
  const S* kb = reinterpret_cast<const S*>(kbv);
  const S* vs = reinterpret_cast<const S*>(vsv);
  const S* vb = reinterpret_cast<const S*>(vbv);
  S* out = reinterpret_cast<S*>(outv);
  constexpr int E = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  constexpr int MAXD = 512;
  __shared__ float qs[MAXD];
  __shared__ float sc[128];
  __shared__ float red[128];

  const int i = blockIdx.x, h = blockIdx.y, b = blockIdx.z, tid = threadIdx.x;
  const int kvh = h / (Hq / Hkv);
  const int G = D / gs;
  const int KW = D / E;
  const int64_t valid = row_valid(geo, b);
  const int64_t base_slot = row_base_slot(geo, b, valid);
  const int64_t rowbase = ((int64_t)b * Hkv + kvh) * geo.cap;
  const int64_t qoff = (((int64_t)b * Hq + h) * Lq + i) * D;
  const float scale_t = Conv<T>::round(scale);
  for (int d = tid; d < D; d += 128) qs[d] = scaled_q<T>(Conv<T>::load(q, qoff + d), scale_t, scale != 1.0f);

  const int64_t pos = valid - Lq + i;
  int64_t jend = valid;
  if (causal && pos + 1 < jend) jend = pos + 1;
  int64_t jbeg = 0;
  if (window > 0 && pos - window + 1 > 0) jbeg = pos - window + 1;
  if (jend < jbeg) jend = jbeg;

  float m_run = -INFINITY, l_run = 0.f;
  float o[MAXD / 128];
#pragma unroll
  for (int k = 0; k < MAXD / 128; k++) o[k] = 0.f;
  __syncthreads();

  const uint8_t* mrow = amask ? amask + (int64_t)b * mask_bs + (int64_t)i * mask_rs : nullptr;
  // o = sum over the keys c0 .. c0 + nkeys - 1 of sc[key] V[key], o scaled by alpha first
  auto accumulate_v = [&](int64_t c0, int nkeys, float alpha) {
#pragma unroll
    for (int k = 0; k < MAXD / 128; k++) {
      const int d = tid + 128 * k;
      if (d < D) {
        float acc = o[k] * alpha;
        for (int jj = 0; jj < nkeys; jj++) {
          const int64_t row = rowbase + slot_of(base_slot, c0 + jj, geo.cap);
          const float cv = (float)((vp[row * KW + d / E] >> (BITS * (d % E))) & MASK);
          const float wv = Conv<T>::load(vs, row * G + d / gs) * cv + Conv<T>::load(vb, row * G + d / gs);
          acc += sc[jj] * wv;
        }
        o[k] = acc;
      }
    }
  };

  for (int64_t c0 = jbeg; c0 < jend; c0 += 128) {
    const int64_t j = c0 + tid;
    const bool attend = j < jend && (!mrow || mrow[j] != 0);
    float s = -INFINITY;
    if (attend) {
      const int64_t row = rowbase + slot_of(base_slot, j, geo.cap);
      const uint32_t* kr = kp + row * KW;
      float acc = 0.f;
      for (int g = 0; g < G; g++) {
        const float sg = Conv<T>::load(ks, row * G + g), bg = Conv<T>::load(kb, row * G + g);
        for (int d = g * gs; d < (g + 1) * gs; d++) {
          const float cv = (float)((kr[d / E] >> (BITS * (d % E))) & MASK);
          acc += qs[d] * (sg * cv + bg);
        }
      }
      s = acc * LOG2E;
    }
    red[tid] = s;
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
      if (tid < st) red[tid] = fmaxf(red[tid], red[tid + st]);
      __syncthreads();
    }
    const float m_new = fmaxf(m_run, red[0]);
    // (a chunk with no attended key leaves m at -inf: nothing to rescale)
    const float alpha = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
    const float pj = attend ? exp2f(s - m_new) : 0.f;
    sc[tid] = pj;
    __syncthreads();
    red[tid] = pj;
    __syncthreads();
    for (int st = 64; st > 0; st >>= 1) {
      if (tid < st) red[tid] += red[tid + st];
      __syncthreads();
    }
    l_run = l_run * alpha + red[0];
    m_run = m_new;
    accumulate_v(c0, (int)min((int64_t)128, jend - c0), alpha);
    __syncthreads();
  }
  if (mrow && l_run == 0.f) {  // every valid key masked (workgroup-uniform): the mean of V
    for (int64_t c0 = 0; c0 < valid; c0 += 128) {
      sc[tid] = 1.0f;
      __syncthreads();
      accumulate_v(c0, (int)min((int64_t)128, valid - c0), 1.0f);
      __syncthreads();
    }
    l_run = (float)valid;
  }
#pragma unroll
  for (int k = 0; k < MAXD / 128; k++) {
    const int d = tid + 128 * k;
    if (d < D) Conv<T>::store(out, qoff + d, l_run > 0.f ? o[k] / l_run : 0.f);
  }
}

// Keys per workgroup: MLXQ_DECODE_CHUNK (a power of two in [32, MAXC]) if
// set, else the largest chunk that still gives every CU a workgroup.
int decode_chunk_override() {
  static const int v = [] {
    const char* e = getenv("MLXQ_DECODE_CHUNK");
    return e ? atoi(e) : 0;
  }();
  return v;
}

template <typename T, int BITS, int D, int GS>
int launch_decode(const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks, const void* kb,
                  const uint32_t* vp, const void* vs, const void* vb, Geometry geo, float scale, void* out,
                  hipStream_t s, const mlxq::Scratch& scr) {
  using SH = DecodeShape<BITS, D, GS>;
  using SH4 = DecodeShape<BITS, D, GS, 4>;
  constexpr int MAXC = SH::MAXC;
  static_assert(SH4::MAXC == MAXC, "the chunk does not depend on the wave count");
  MLXQ_CHECK(geo.cap * (int64_t)SH::KW * 4 < ((int64_t)1 << 31), "kv cache rows too long for one launch");
  const int64_t cus = mlxq::device_cu_count();
  const int64_t span = geo.valid_len ? geo.cap : geo.n_kv;  // per-row upper bound on keys
  int chunk = MAXC;
  const int ov = decode_chunk_override();
  if (ov >= 32 && ov <= MAXC && (ov & (ov - 1)) == 0) {
    chunk = ov;
  } else {
    // halve the chunk while the launch leaves CUs without a workgroup, down
    // to 128 keys, 64 at 8 bits and D <= 128 (the 1k fp16 8-bit decode: 8.47
    // -> 8.22 us on MI355X; 4-bit and D 256 small grids measured slower at 64)
    const int cmin = (BITS == 8 && D <= 128) ? 64 : 128;
    while (chunk > cmin && ((span + chunk - 1) / chunk) * B * Hkv < cus) chunk /= 2;
  }
  // a ring row's window may start mid-chunk at the wrap point: one extra chunk
  MLXQ_CHECK((chunk & (chunk - 1)) == 0, "decode chunk must be a power of two");
  const int64_t nchunks = (span > 0 ? (span + chunk - 1) / chunk : 1) + (geo.ring_off ? 1 : 0);
  MLXQ_CHECK(nchunks < 65536, "kv length too large for one launch");
  void* pws = nullptr;
  const int nrep = Hq / Hkv;
  const size_t slots = (size_t)B * Hkv * nchunks;
  const size_t obytes = (slots * nrep * D * sizeof(float) + 255) & ~(size_t)255;
  const size_t pbytes = nchunks > 1 ? obytes + slots * nrep * sizeof(float2) : 0;
  if (pbytes) {
    int rc = scr.get(pbytes, &pws, s);
    if (rc) return rc;
  }
  float* part_o = (float*)pws;
  float2* part_ml = pbytes ? (float2*)((uint8_t*)pws + obytes) : nullptr;
  dim3 grid((unsigned)nchunks, (unsigned)Hkv, (unsigned)B);
  // 4-bit D 256 (200+ VGPRs: one 8-wave workgroup a CU) with at least two
  // workgroups a CU: 4-wave workgroups, two a CU (the 32-row batched ring
  // decode, 1280 workgroups: 84-88 -> 67-73 us on MI355X, one box)
  if constexpr (BITS == 4 && D == 256) {
    if (slots >= 2 * (size_t)cus) {
      hipLaunchKernelGGL((sdpa_decode_mfma_kernel<T, BITS, D, GS, 4>), grid, dim3(SH4::NW * 64), 0, s,
                         (const uint16_t*)q, kp, (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs,
                         (const uint16_t*)vb, Hq, Hkv, geo, scale, chunk, (uint16_t*)out, part_o, part_ml);
      MLXQ_LAUNCHED("sdpa_decode_mfma_kernel");
    } else {
      hipLaunchKernelGGL((sdpa_decode_mfma_kernel<T, BITS, D, GS, 8>), grid, dim3(SH::NW * 64), 0, s,
                         (const uint16_t*)q, kp, (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs,
                         (const uint16_t*)vb, Hq, Hkv, geo, scale, chunk, (uint16_t*)out, part_o, part_ml);
      MLXQ_LAUNCHED("sdpa_decode_mfma_kernel");
    }
  } else {
    hipLaunchKernelGGL((sdpa_decode_mfma_kernel<T, BITS, D, GS, 8>), grid, dim3(SH::NW * 64), 0, s, (const uint16_t*)q,
                       kp, (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs, (const uint16_t*)vb, Hq,
                       Hkv, geo, scale, chunk, (uint16_t*)out, part_o, part_ml);
    MLXQ_LAUNCHED("sdpa_decode_mfma_kernel");
  }
  if (nchunks > 1) {
    const int cols = nrep * D / 4;
    dim3 mgrid((unsigned)((cols + 63) / 64), (unsigned)Hkv, (unsigned)B);
    return launch_merge<T>(mgrid, nchunks, s, part_o, part_ml, Hq, Hkv, D, geo, chunk, (uint16_t*)out);
  }
  return MLXQ_OK;
}

template <typename T, int BITS>
int launch_decode_d(int D, int gs, const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks,
                    const void* kb, const uint32_t* vp, const void* vs, const void* vb, Geometry geo, float scale,
                    void* out, hipStream_t s, const mlxq::Scratch& scr) {
#define DEC(DV, GV)                                                                                             \
  if (D == DV && gs == GV)                                                                                      \
    return launch_decode<T, BITS, DV, GV>(q, B, Hq, Hkv, kp, ks, kb, vp, vs, vb, geo, scale, out, s, scr);
  DEC(128, 32) DEC(128, 64) DEC(128, 128)
  DEC(256, 32) DEC(256, 64) DEC(256, 128)
  if constexpr (BITS == 8) {
    DEC(64, 32) DEC(64, 64)
  }
#undef DEC
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "decode: no MFMA instance for this head_dim/group_size");
}

template <typename T, int BITS, int D, int GS>
int launch_decode_wide(const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks, const void* kb,
                       const uint32_t* vp, const void* vs, const void* vb, Geometry geo, float scale, void* out,
                       hipStream_t s, const mlxq::Scratch& scr) {
  using SH = WideShape<D, GS, BITS>;
  MLXQ_CHECK(geo.cap * (int64_t)SH::KW * 4 < ((int64_t)1 << 31), "kv cache rows too long for one launch");
  const int64_t span = geo.valid_len ? geo.cap : geo.n_kv;  // per-row upper bound on keys
  int chunk = SH::MAXC;
  const int ov = decode_chunk_override();
  if (ov >= SH::TK && ov <= SH::MAXC && (ov & (ov - 1)) == 0) {
    chunk = ov;
  } else {
    const int64_t cus = mlxq::device_cu_count();
    while (chunk > SH::TK && ((span + chunk - 1) / chunk) * B * Hkv < cus) chunk /= 2;
  }
  MLXQ_CHECK((chunk & (chunk - 1)) == 0, "decode chunk must be a power of two");
  const int64_t nchunks = (span > 0 ? (span + chunk - 1) / chunk : 1) + (geo.ring_off ? 1 : 0);
  MLXQ_CHECK(nchunks < 65536, "kv length too large for one launch");
  void* pws = nullptr;
  const int nrep = Hq / Hkv;
  const size_t slots = (size_t)B * Hkv * nchunks;
  const size_t obytes = (slots * nrep * D * sizeof(float) + 255) & ~(size_t)255;
  const size_t pbytes = nchunks > 1 ? obytes + slots * nrep * sizeof(float2) : 0;
  if (pbytes) {
    int rc = scr.get(pbytes, &pws, s);
    if (rc) return rc;
  }
  float* part_o = (float*)pws;
  float2* part_ml = pbytes ? (float2*)((uint8_t*)pws + obytes) : nullptr;
  dim3 grid((unsigned)nchunks, (unsigned)Hkv, (unsigned)B);
  hipLaunchKernelGGL((sdpa_decode_wide_kernel<T, BITS, D, GS>), grid, dim3(SH::NW * 64), 0, s, (const uint16_t*)q,
                     kp, (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs, (const uint16_t*)vb, Hq,
                     Hkv, geo, scale, chunk, (uint16_t*)out, part_o, part_ml);
  MLXQ_LAUNCHED("sdpa_decode_wide_kernel");
  if (nchunks > 1) {
    const int cols = nrep * D / 4;
    dim3 mgrid((unsigned)((cols + 63) / 64), (unsigned)Hkv, (unsigned)B);
    return launch_merge<T>(mgrid, nchunks, s, part_o, part_ml, Hq, Hkv, D, geo, chunk, (uint16_t*)out);
  }
  return MLXQ_OK;
}

template <typename T, int BITS>
int launch_decode_wide_d(int D, int gs, const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks,
                         const void* kb, const uint32_t* vp, const void* vs, const void* vb, Geometry geo,
                         float scale, void* out, hipStream_t s, const mlxq::Scratch& scr) {
#define WDEC(DV, GV)                                                                                            \
  if (D == DV && gs == GV)                                                                                      \
    return launch_decode_wide<T, BITS, DV, GV>(q, B, Hq, Hkv, kp, ks, kb, vp, vs, vb, geo, scale, out, s, scr);
  WDEC(128, 32) WDEC(128, 64) WDEC(128, 128)
  WDEC(256, 32) WDEC(256, 64) WDEC(256, 128)
  WDEC(512, 64) WDEC(512, 128)
#undef WDEC
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "decode: no wide MFMA instance for this head_dim/group_size");
}

// The wide decode kernel: up to 16 query heads per kv head, at most 8
// quant groups per row (one row's K scales are one 2G-byte load; V scales
// are read as aligned dwords).
bool decode_wide_ok(int dtype, int bits, int D, int gs, int nrep, std::initializer_list<const void*> sb) {
  if (!mlxq::is_half_dtype(dtype)) return false;
  if (bits != 4 && bits != 8) return false;
  if (!(D == 128 || D == 256 || (D == 512 && gs >= 64))) return false;
  const uintptr_t al = 2 * (D / gs) > 4 ? 2 * (D / gs) : 4;
  for (const void* p : sb)
    if ((uintptr_t)p % al) return false;
  return nrep <= 16;
}

// The MFMA decode kernel reads a cache row's G = D/gs scales (biases) with
// one 2G-byte load, so those arrays must be 2G-byte aligned.
bool decode_mfma_ok(int dtype, int bits, int D, int gs, int nrep, std::initializer_list<const void*> sb) {
  if (!mlxq::is_half_dtype(dtype)) return false;
  if (bits != 4 && bits != 8) return false;
  const bool dok = D == 128 || D == 256 || (bits == 8 && D == 64 && gs <= 64);
  if (!dok) return false;
  for (const void* p : sb)
    if ((uintptr_t)p % (2 * (D / gs))) return false;
  return nrep * (D / gs) <= 16;
}

// The whole dispatch of mlxq_quantized_sdpa, with its scratch (split-K
// partials) taken from `scr`.
// the generic kernel (every geometry, mask and dtype), with an optional
// array mask
int launch_generic(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D, const uint32_t* k_packed,
                   const void* k_scales, const void* k_biases, const uint32_t* v_packed, const void* v_scales,
                   const void* v_biases, Geometry geo, int causal, int window, float scale, int group_size, int bits,
                   void* out, hipStream_t s, const uint8_t* amask, int64_t mask_bs, int64_t mask_rs) {
  dim3 grid((unsigned)Lq, (unsigned)Hq, (unsigned)B);
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 2>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out,
                           amask, mask_bs, mask_rs);
        break;
      case 4:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 4>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out,
                           amask, mask_bs, mask_rs);
        break;
      default:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 8>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out,
                           amask, mask_bs, mask_rs);
        break;
    }
  });
  MLXQ_LAUNCHED("sdpa_generic_kernel");
  return MLXQ_OK;
}

// argument checks shared by the entry points (buffers only when there is
// work: an empty batch, head or query extent is a no-op)
int check_sdpa_args(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D, const uint32_t* k_packed,
                    const void* k_scales, const void* k_biases, const uint32_t* v_packed, const void* v_scales,
                    const void* v_biases, int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                    const int32_t* ring_offset, int group_size, int bits, const void* out) {
  MLXQ_REQUIRE_INIT();
  MLXQ_CHECK(mlxq::dtype_supported(dtype), "dtype must be float16, bfloat16 or float32");
  MLXQ_CHECK(bits == 2 || bits == 4 || bits == 8, "bits must be 2, 4 or 8");
  MLXQ_CHECK(group_size == 32 || group_size == 64 || group_size == 128, "group_size must be 32, 64 or 128");
  MLXQ_CHECK(B >= 0 && Hq >= 0 && Hkv > 0 && Lq >= 0, "bad batch/head/query extents");
  MLXQ_CHECK(Hq % Hkv == 0, "query heads must be a multiple of kv heads");
  MLXQ_CHECK(D > 0 && D % group_size == 0 && D <= 512, "head_dim must be a multiple of group_size, <= 512");
  MLXQ_CHECK(kv_capacity > 0, "kv_capacity must be positive");
  MLXQ_CHECK(valid_len || (n_kv >= 0 && n_kv <= kv_capacity), "n_kv must lie in [0, kv_capacity]");
  MLXQ_CHECK(!ring_offset || valid_len, "ring_offset requires valid_len");
  if (B == 0 || Hq == 0 || Lq == 0) return MLXQ_OK;
  MLXQ_CHECK(q && k_packed && k_scales && k_biases && v_packed && v_scales && v_biases && out, "null buffer");
  MLXQ_CHECK((uintptr_t)q % 16 == 0 && (uintptr_t)k_packed % 16 == 0 && (uintptr_t)v_packed % 16 == 0,
             "q and packed caches must be 16-byte aligned");
  return MLXQ_OK;
}

int sdpa_dispatch(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D, const uint32_t* k_packed,
                  const void* k_scales, const void* k_biases, const uint32_t* v_packed, const void* v_scales,
                  const void* v_biases, int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                  const int32_t* ring_offset, int mask_mode, int window, float scale, int group_size, int bits,
                  void* out, void* stream, const mlxq::Scratch& scr) {
  int rc = check_sdpa_args(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                           kv_capacity, n_kv, valid_len, ring_offset, group_size, bits, out);
  if (rc) return rc;
  MLXQ_CHECK(mask_mode == MLXQ_MASK_NONE || mask_mode == MLXQ_MASK_CAUSAL, "unknown mask mode");
  MLXQ_CHECK(window >= 0, "negative window");
  if (B == 0 || Hq == 0 || Lq == 0) return MLXQ_OK;
  hipStream_t s = mlxq::resolve_stream(stream);
  Geometry geo{kv_capacity, valid_len ? kv_capacity : n_kv, valid_len, ring_offset};
  const int nrep = Hq / Hkv;
  // Lq = 1 attends every valid key under either mask (its position is the last one)
  const bool decode = Lq == 1 && (mask_mode == MLXQ_MASK_NONE || window == 0);
  if (decode && decode_mfma_ok(dtype, bits, D, group_size, nrep, {k_scales, k_biases, v_scales, v_biases})) {
    if (dtype == MLXQ_BFLOAT16)
      return bits == 4 ? launch_decode_d<BF16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                  v_packed, v_scales, v_biases, geo, scale, out, s, scr)
                       : launch_decode_d<BF16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                  v_packed, v_scales, v_biases, geo, scale, out, s, scr);
    return bits == 4 ? launch_decode_d<F16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases, v_packed,
                                               v_scales, v_biases, geo, scale, out, s, scr)
                     : launch_decode_d<F16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases, v_packed,
                                               v_scales, v_biases, geo, scale, out, s, scr);
  }
  if (decode && decode_wide_ok(dtype, bits, D, group_size, nrep, {k_scales, k_biases, v_scales, v_biases})) {
    if (dtype == MLXQ_BFLOAT16)
      return bits == 4 ? launch_decode_wide_d<BF16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                       v_packed, v_scales, v_biases, geo, scale, out, s, scr)
                       : launch_decode_wide_d<BF16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                       v_packed, v_scales, v_biases, geo, scale, out, s, scr);
    return bits == 4 ? launch_decode_wide_d<F16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                    v_packed, v_scales, v_biases, geo, scale, out, s, scr)
                     : launch_decode_wide_d<F16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                    v_packed, v_scales, v_biases, geo, scale, out, s, scr);
  }
  const int causal = mask_mode == MLXQ_MASK_CAUSAL;
  // Lq > 1 on the matrix cores: plain (non-ring) caches, T = bf16/f16, 4/8-bit
  const bool prefill_ok = Lq > 1 && !ring_offset && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                          (D == 64 || D == 128) && (uintptr_t)k_scales % 2 == 0 &&
                          kv_capacity * (int64_t)D * bits / 8 < ((int64_t)1 << 31);
  if (prefill_ok) {
    if (dtype == MLXQ_BFLOAT16)
      return bits == 4 ? launch_prefill<BF16, 4>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                 v_packed, v_scales, v_biases, geo, causal, window, scale, out, s)
                       : launch_prefill<BF16, 8>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                 v_packed, v_scales, v_biases, geo, causal, window, scale, out, s);
    return bits == 4 ? launch_prefill<F16, 4>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases, v_packed,
                                              v_scales, v_biases, geo, causal, window, scale, out, s)
                     : launch_prefill<F16, 8>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases, v_packed,
                                              v_scales, v_biases, geo, causal, window, scale, out, s);
  }
  // head_dim 256 / 512 (one row's K scales as aligned dwords)
  const bool prefill_wide_ok = Lq > 1 && !ring_offset && mlxq::is_half_dtype(dtype) && (bits == 4 || bits == 8) &&
                               (D == 256 || (D == 512 && group_size >= 64)) && (uintptr_t)k_scales % 4 == 0 &&
                               (uintptr_t)k_biases % 4 == 0 && (uintptr_t)v_scales % 4 == 0 &&
                               (uintptr_t)v_biases % 4 == 0 &&
                               kv_capacity * (int64_t)D * bits / 8 < ((int64_t)1 << 31);
  if (prefill_wide_ok) {
    if (dtype == MLXQ_BFLOAT16)
      return bits == 4 ? launch_prefill_wide<BF16, 4>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                      v_packed, v_scales, v_biases, geo, causal, window, scale, out, s, scr)
                       : launch_prefill_wide<BF16, 8>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                      v_packed, v_scales, v_biases, geo, causal, window, scale, out, s, scr);
    return bits == 4 ? launch_prefill_wide<F16, 4>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                   v_packed, v_scales, v_biases, geo, causal, window, scale, out, s, scr)
                     : launch_prefill_wide<F16, 8>(D, group_size, q, B, Hq, Hkv, Lq, k_packed, k_scales, k_biases,
                                                   v_packed, v_scales, v_biases, geo, causal, window, scale, out, s, scr);
  }
  return launch_generic(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases, geo,
                        causal, window, scale, group_size, bits, out, s, nullptr, 0, 0);
}

}  // namespace

extern "C" int mlxq_quantized_sdpa(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                   const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                   const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                   int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                   const int32_t* ring_offset, int mask_mode, int window, float scale,
                                   int group_size, int bits, void* out, void* stream) {
  return sdpa_dispatch(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                       kv_capacity, n_kv, valid_len, ring_offset, mask_mode, window, scale, group_size, bits, out,
                       stream, mlxq::Scratch{});
}

extern "C" int mlxq_quantized_sdpa_noalloc(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                           const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                           const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                           int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                           const int32_t* ring_offset, int mask_mode, int window, float scale,
                                           int group_size, int bits, void* out, void* stream) {
  MLXQ_REQUIRE_INIT();
  mlxq::Scratch scr;
  const int rc = mlxq::noalloc_scratch(&scr);
  if (rc) return rc;
  return sdpa_dispatch(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases,
                       kv_capacity, n_kv, valid_len, ring_offset, mask_mode, window, scale, group_size, bits, out,
                       stream, scr);
}

extern "C" int mlxq_quantized_sdpa_array_mask(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                              const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                              const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                              int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                              const int32_t* ring_offset, const uint8_t* mask,
                                              int64_t mask_batch_stride, int64_t mask_row_stride, float scale,
                                              int group_size, int bits, void* out, void* stream) {
  const int rc = check_sdpa_args(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales,
                                 v_biases, kv_capacity, n_kv, valid_len, ring_offset, group_size, bits, out);
  if (rc) return rc;
  MLXQ_CHECK(mask_batch_stride >= 0, "negative mask batch stride");
  // a row's keys are logical positions 0 .. valid - 1 <= n_kv (kv_capacity with valid_len)
  MLXQ_CHECK(mask_row_stride >= (valid_len ? kv_capacity : n_kv), "mask rows must cover every key");
  if (B == 0 || Hq == 0 || Lq == 0) return MLXQ_OK;
  MLXQ_CHECK(mask, "null mask");
  Geometry geo{kv_capacity, valid_len ? kv_capacity : n_kv, valid_len, ring_offset};
  return launch_generic(q, dtype, B, Hq, Hkv, Lq, D, k_packed, k_scales, k_biases, v_packed, v_scales, v_biases, geo,
                        0, 0, scale, group_size, bits, out, mlxq::resolve_stream(stream), mask, mask_batch_stride,
                        mask_row_stride);
}
