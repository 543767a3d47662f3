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
// Waves merge through LDS; chunks of one (b, kv head) merge in the last
// workgroup to arrive (fixed order, deterministic).  Key chunk geometry
// handles the rotating caches' ring (slot = (ring_off - valid + j) mod cap).
//
// Everything the MFMA decode kernel does not cover (Lq > 1, D = 512 or
// nRep * D/gs > 16, 2-bit, fp32) runs a generic VALU kernel with the same
// semantics.
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
  int64_t s = ((int64_t)g.ring_off[b] - valid) % g.cap;
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

template <typename T, int BITS, int D, int GS, int TPW>
__global__ void __launch_bounds__(256) sdpa_decode_mfma_kernel(
    const uint16_t* __restrict__ q, const uint32_t* __restrict__ kp, const uint16_t* __restrict__ ksc,
    const uint16_t* __restrict__ kbi, const uint32_t* __restrict__ vp, const uint16_t* __restrict__ vsc,
    const uint16_t* __restrict__ vbi, int Hq, int Hkv, Geometry geo, float scale, int chunk,
    uint16_t* __restrict__ out, float* __restrict__ part, uint32_t* __restrict__ counters) {
  using CO = CodeOps<T, BITS>;
  constexpr int G = D / GS;
  constexpr int KW = D * BITS / 32;  // packed words per cache row
  constexpr int LKW = KW / 4;        // K-side words per lane (a quarter row)
  constexpr int WPS = BITS / 4;      // K-side words per k-step
  constexpr int KSTEPS = D / 32;
  constexpr int VM = KW / 16;        // V-side word columns per lane
  constexpr int E = 32 / BITS;       // codes per word
  constexpr int DT = D / 16;         // V-side MFMA tiles
  constexpr int MAXC = 128 * TPW;    // keys per workgroup
  static_assert(VM * E == DT, "tile bookkeeping");

  __shared__ float sb_lds[4][G][MAXC];  // K scale, K bias, V scale, V bias
  __shared__ float u_lds[4][16 * GS];   // per-wave unnormalised outputs [wave][h*D + d] (nrep*D <= 16*GS)
  __shared__ float m_lds[4][16], l_lds[4][16];
  __shared__ uint32_t last_flag;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ln = lane & 15, lg = lane >> 4;
  const int b = blockIdx.z, kvh = blockIdx.y, c = blockIdx.x;
  const int nrep = Hq / Hkv;
  const int R = nrep * G;

  const int64_t valid = row_valid(geo, b);
  const int nch = (int)((valid + chunk - 1) / chunk);
  if (c > 0 && c >= nch) return;
  const int64_t out_base = ((int64_t)b * Hq + (int64_t)kvh * nrep) * D;
  if (nch == 0) {  // nothing to attend: zeros (no counter traffic)
    for (int i = tid; i < nrep * D; i += 256) out[out_base + i] = 0;
    return;
  }
  const int64_t j0 = (int64_t)c * chunk;
  const int nk = (int)min((int64_t)chunk, valid - j0);
  const int64_t base_slot = row_base_slot(geo, b, valid);
  const int64_t rowbase = ((int64_t)b * Hkv + kvh) * geo.cap;

  // ---- stage this chunk's scales/biases as float, layout [array][g][key];
  // slots past the chunk's last key read as 0 so masked keys stay finite
  {
    const uint16_t* arrs[4] = {ksc, kbi, vsc, vbi};
    constexpr int per = MAXC * G;
    for (int idx = tid; idx < 4 * per; idx += 256) {
      const int a = idx / per, e = idx % per, key = e / G, g = e % G;
      float val = 0.f;
      if (key < nk) {
        const int64_t row = rowbase + slot_of(base_slot, j0 + key, geo.cap);
        val = Conv<T>::from_bits(arrs[a][row * G + g]);
      }
      sb_lds[a][g][key] = val;
    }
  }

  // ---- q' operand (B of the score MFMA): column ln = (g, h) ---------------
  const int r_me = ln;
  const bool r_ok = r_me < R;
  const int g_me = r_ok ? r_me / nrep : G - 1;
  const int h_me = r_ok ? r_me % nrep : 0;
  const float scale_t = Conv<T>::round(scale);
  const bool apply_scale = scale != 1.0f;
  u32x4_t qop[KSTEPS];
  float qsum = 0.f;
  {
    const uint16_t* qrow = q + out_base + (int64_t)h_me * D;
#pragma unroll
    for (int j = 0; j < KSTEPS; j++) {
      const int d0 = lg * (D / 4) + 8 * j;
      const bool in_group = r_ok && (d0 / GS == g_me);
      u32x4_t raw = *reinterpret_cast<const u32x4_t*>(qrow + d0);
      uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int p = 0; p < 4; p++) {
        const float lo = scaled_q<T>(Conv<T>::from_bits(wv[p] & 0xffffu), scale_t, apply_scale);
        const float hi = scaled_q<T>(Conv<T>::from_bits(wv[p] >> 16), scale_t, apply_scale);
        wv[p] = in_group ? Mma<T>::pack2(lo, hi) : 0u;
        qsum += in_group ? lo + hi : 0.f;
      }
      qop[j] = permute8<CO::ORDER>(u32x4_t{wv[0], wv[1], wv[2], wv[3]});
    }
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
  }
  __syncthreads();  // sb_lds ready

  // ---- issue every load of this wave's tiles up front ---------------------
  // tile t of this wave covers chunk keys [(wave + 4t) * 32, +32)
  uint32_t kreg[TPW][2][LKW];
  uint32_t vreg[TPW][8][VM];
#pragma unroll
  for (int t = 0; t < TPW; t++) {
    const int kt = (wave + 4 * t) * 32;
    if (kt < nk) {
#pragma unroll
      for (int sub = 0; sub < 2; sub++) {
        int key = kt + 16 * sub + ln;
        key = key < nk ? key : nk - 1;
        const uint32_t* src = kp + (rowbase + slot_of(base_slot, j0 + key, geo.cap)) * KW + lg * LKW;
#pragma unroll
        for (int w4 = 0; w4 < LKW; w4 += 4) {
          if constexpr (LKW >= 4) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + w4);
            kreg[t][sub][w4] = v.x;
            kreg[t][sub][w4 + 1] = v.y;
            kreg[t][sub][w4 + 2] = v.z;
            kreg[t][sub][w4 + 3] = v.w;
          }
        }
        if constexpr (LKW == 2) {
          const uint2 v = *reinterpret_cast<const uint2*>(src);
          kreg[t][sub][0] = v.x;
          kreg[t][sub][1] = v.y;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        int key = kt + (e < 4 ? 4 * lg + e : 16 + 4 * lg + (e - 4));
        key = key < nk ? key : nk - 1;
        const uint32_t* src = vp + (rowbase + slot_of(base_slot, j0 + key, geo.cap)) * KW;
#pragma unroll
        for (int m = 0; m < VM; m++) vreg[t][e][m] = src[16 * m + ln];
      }
    }
  }

  // ---- per-wave online softmax state --------------------------------------
  float m_run = -INFINITY;  // per head h_me (log2 domain), replicated over g and lane groups
  float l_run = 0.f;        // partial over this lane's keys
  float sp_run = 0.f;       // sum of T(p * s_v) over this lane's k slots, row r_me
  float pb_run = 0.f;       // sum of p * b_v over this lane's keys, row r_me
  f32x4_t oacc[DT];
#pragma unroll
  for (int i = 0; i < DT; i++) oacc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < TPW; t++) {
    const int kt = (wave + 4 * t) * 32;
    if (kt >= nk) continue;  // wave-uniform

    // scores: two 16-key sub-tiles, D/32 k-steps each
    f32x4_t sacc[2];
#pragma unroll
    for (int sub = 0; sub < 2; sub++) {
      f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < KSTEPS; j++) {
        u32x4_t a;
        if constexpr (BITS == 4)
          a = CodeOps<T, 4>::operand(kreg[t][sub][j * WPS]);
        else
          a = CodeOps<T, BITS>::operand(kreg[t][sub][j * WPS], kreg[t][sub][j * WPS + WPS - 1]);
        acc = Mma<T>::mma(a, qop[j], acc);
      }
      sacc[sub] = acc;
    }

    // key e of this lane: e<4 -> kt + 4lg + e, e>=4 -> kt + 16 + 4lg + (e-4)
    float s2[8];
    float kscale[8], kbias[8];
    {
      const float4 s_a = *reinterpret_cast<const float4*>(&sb_lds[0][g_me][kt + 4 * lg]);
      const float4 s_b = *reinterpret_cast<const float4*>(&sb_lds[0][g_me][kt + 16 + 4 * lg]);
      const float4 b_a = *reinterpret_cast<const float4*>(&sb_lds[1][g_me][kt + 4 * lg]);
      const float4 b_b = *reinterpret_cast<const float4*>(&sb_lds[1][g_me][kt + 16 + 4 * lg]);
      kscale[0] = s_a.x; kscale[1] = s_a.y; kscale[2] = s_a.z; kscale[3] = s_a.w;
      kscale[4] = s_b.x; kscale[5] = s_b.y; kscale[6] = s_b.z; kscale[7] = s_b.w;
      kbias[0] = b_a.x; kbias[1] = b_a.y; kbias[2] = b_a.z; kbias[3] = b_a.w;
      kbias[4] = b_b.x; kbias[5] = b_b.y; kbias[6] = b_b.z; kbias[7] = b_b.w;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const float cdot = e < 4 ? sacc[0][e] : sacc[1][e - 4];
      // this quant group's part of the score of key e for head h_me
      float part_g = kscale[e] * cdot + (kbias[e] - CO::OFFSET * kscale[e]) * qsum;
      // sum over groups: columns (g', h_me) of this lane's 16-lane row
      float tot = 0.f;
#pragma unroll
      for (int gg = 0; gg < G; gg++) tot += __shfl(part_g, (lane & 48) + gg * nrep + h_me);
      const int key = kt + (e < 4 ? 4 * lg + e : 12 + 4 * lg + e);
      s2[e] = key < nk ? tot * LOG2E : -INFINITY;
    }

    // online softmax over this tile's 32 keys
    float tmax = s2[0];
#pragma unroll
    for (int e = 1; e < 8; e++) tmax = fmaxf(tmax, s2[e]);
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    // Lazy rescale: keep the reference max unless this tile exceeds it by
    // more than 2^8 (p stays <= 256, fp32 and T both hold that exactly as a
    // scale); the accumulators are only rewritten when it moves.
    const float m_new = tmax > m_run + 8.0f ? tmax : m_run;  // first tile: m_run = -inf
    const float alpha = exp2f(m_run - m_new);                 // 1 unless moved; -inf -> 0
    m_run = m_new;
    float p[8];
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      p[e] = exp2f(s2[e] - m_new);
      psum += p[e];
    }
    l_run = l_run * alpha + psum;

    // value-side A operand: row (g_me, h_me) = p * s_v, rounded to T
    float vscale[8], vbias[8];
    {
      const float4 s_a = *reinterpret_cast<const float4*>(&sb_lds[2][g_me][kt + 4 * lg]);
      const float4 s_b = *reinterpret_cast<const float4*>(&sb_lds[2][g_me][kt + 16 + 4 * lg]);
      const float4 b_a = *reinterpret_cast<const float4*>(&sb_lds[3][g_me][kt + 4 * lg]);
      const float4 b_b = *reinterpret_cast<const float4*>(&sb_lds[3][g_me][kt + 16 + 4 * lg]);
      vscale[0] = s_a.x; vscale[1] = s_a.y; vscale[2] = s_a.z; vscale[3] = s_a.w;
      vscale[4] = s_b.x; vscale[5] = s_b.y; vscale[6] = s_b.z; vscale[7] = s_b.w;
      vbias[0] = b_a.x; vbias[1] = b_a.y; vbias[2] = b_a.z; vbias[3] = b_a.w;
      vbias[4] = b_b.x; vbias[5] = b_b.y; vbias[6] = b_b.z; vbias[7] = b_b.w;
    }
    uint32_t aw[4];
    float spt = 0.f, pbt = 0.f;
#pragma unroll
    for (int pr = 0; pr < 4; pr++) {
      const float x0 = Conv<T>::round(p[2 * pr] * vscale[2 * pr]);
      const float x1 = Conv<T>::round(p[2 * pr + 1] * vscale[2 * pr + 1]);
      aw[pr] = Mma<T>::pack2(x0, x1);
      spt += x0 + x1;
      pbt += p[2 * pr] * vbias[2 * pr] + p[2 * pr + 1] * vbias[2 * pr + 1];
    }
    sp_run = sp_run * alpha + spt;
    pb_run = pb_run * alpha + pbt;
    const u32x4_t aop = {aw[0], aw[1], aw[2], aw[3]};

    // rescale the accumulator rows (4lg + i) by their head's alpha
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float ai = __shfl(alpha, 4 * lg + i);
#pragma unroll
        for (int tt = 0; tt < DT; tt++) oacc[tt][i] *= ai;
      }
    }

    // value MFMAs: tile (m, e') covers d = (16m + ln) * E + e'
#pragma unroll
    for (int m = 0; m < VM; m++) {
      if constexpr (BITS == 4) {
        uint32_t plo[4], phi[4];
#pragma unroll
        for (int pr = 0; pr < 4; pr++) {
          plo[pr] = perm_b32(vreg[t][2 * pr + 1][m], vreg[t][2 * pr][m], 0x05040100u);
          phi[pr] = perm_b32(vreg[t][2 * pr + 1][m], vreg[t][2 * pr][m], 0x07060302u);
        }
#pragma unroll
        for (int ep = 0; ep < 8; ep++) {
          const int sh = 4 * (ep & 3);
          u32x4_t bop;
          bop.x = (((ep < 4 ? plo[0] : phi[0]) >> sh) & 0x000f000fu) | Mma<T>::MAGIC;
          bop.y = (((ep < 4 ? plo[1] : phi[1]) >> sh) & 0x000f000fu) | Mma<T>::MAGIC;
          bop.z = (((ep < 4 ? plo[2] : phi[2]) >> sh) & 0x000f000fu) | Mma<T>::MAGIC;
          bop.w = (((ep < 4 ? plo[3] : phi[3]) >> sh) & 0x000f000fu) | Mma<T>::MAGIC;
          oacc[m * E + ep] = Mma<T>::mma(aop, bop, oacc[m * E + ep]);
        }
      } else {
#pragma unroll
        for (int ep = 0; ep < 4; ep++) {
          uint32_t bw[4];
#pragma unroll
          for (int pr = 0; pr < 4; pr++) {
            const uint32_t wa = vreg[t][2 * pr][m], wb = vreg[t][2 * pr + 1][m];
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
  }

  // ---- wave result: u[h][d] = O - off * sp + pb (rows whose group owns d) -
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  sp_run += __shfl_xor(sp_run, 16);
  sp_run += __shfl_xor(sp_run, 32);
  pb_run += __shfl_xor(pb_run, 16);
  pb_run += __shfl_xor(pb_run, 32);
  constexpr float VOFF = CodeOps<T, BITS>::OFFSET;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * lg + i;
    const float sp_r = __shfl(sp_run, r);
    const float pb_r = __shfl(pb_run, r);
    if (r < R) {
      const int g = r / nrep, h = r % nrep;
#pragma unroll
      for (int tt = 0; tt < DT; tt++) {
        const int m = tt / E, ep = tt % E;
        const int d = (16 * m + ln) * E + ep;
        if (d / GS == g) u_lds[wave][h * D + d] = oacc[tt][i] - VOFF * sp_r + pb_r;
      }
    }
  }
  if (lane < nrep) {
    m_lds[wave][lane] = m_run;  // lane < nrep has h_me = lane (group 0)
    l_lds[wave][lane] = l_run;
  }
  __syncthreads();

  // ---- merge the four waves ----------------------------------------------
  const bool single = nch == 1;
  const int64_t pstride = (int64_t)nrep * (D + 2);
  float* mypart = part + (((int64_t)b * Hkv + kvh) * gridDim.x + c) * pstride;
  for (int idx = tid; idx < nrep * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; w++) M = fmaxf(M, m_lds[w][h]);
    float U = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
      const float f = exp2f(m_lds[w][h] - M);  // empty wave: m = -inf -> 0
      if (f > 0.f) {
        U += f * u_lds[w][idx];
        L += f * l_lds[w][h];
      }
    }
    if (single) {
      Conv<T>::store(out, out_base + idx, U / L);
    } else {
      mypart[h * (D + 2) + d] = U;
      if (d == 0) {
        mypart[h * (D + 2) + D] = M;
        mypart[h * (D + 2) + D + 1] = L;
      }
    }
  }
  if (single) return;

  // ---- last chunk to arrive merges all chunks of this (b, kv head) -------
  // One release RMW per workgroup publishes its partial (the barrier makes
  // every thread's stores part of thread 0's release); only the merging
  // workgroup pays the acquire.  No full fence: that would invalidate the L2
  // under every other workgroup still streaming K/V.
  __syncthreads();
  if (tid == 0) {
    uint32_t* ctr = counters + (int64_t)b * Hkv + kvh;
    const uint32_t prev = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (uint32_t)(nch - 1);
    if (last_flag) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
  if (!last_flag) return;
  const float* parts = part + ((int64_t)b * Hkv + kvh) * gridDim.x * pstride;
  for (int idx = tid; idx < nrep * D; idx += 256) {
    const int h = idx / D, d = idx % D;
    float M = -INFINITY;
    for (int cc = 0; cc < nch; cc++) M = fmaxf(M, parts[cc * pstride + h * (D + 2) + D]);
    float U = 0.f, L = 0.f;
    for (int cc = 0; cc < nch; cc++) {
      const float* pc = parts + cc * pstride + h * (D + 2);
      const float f = exp2f(pc[D] - M);
      U += f * pc[d];
      L += f * pc[D + 1];
    }
    Conv<T>::store(out, out_base + idx, U / L);
  }
}

// ========================================================== generic kernel
// One workgroup (128 threads) per (batch row, q head, query).  Scores for
// 128 keys at a time (one key per thread, fp32 dot of fp32-dequantized K),
// online softmax through LDS, values accumulated with threads over d.
template <typename T, int BITS>
__global__ void __launch_bounds__(128) sdpa_generic_kernel(
    const void* __restrict__ qv, const uint32_t* __restrict__ kp, const void* __restrict__ ksv,
    const void* __restrict__ kbv, const uint32_t* __restrict__ vp, const void* __restrict__ vsv,
    const void* __restrict__ vbv, int Hq, int Hkv, int Lq, int D, int gs, Geometry geo, int causal, int window,
    float scale, void* __restrict__ outv) {
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

  for (int64_t c0 = jbeg; c0 < jend; c0 += 128) {
    const int64_t j = c0 + tid;
    float s = -INFINITY;
    if (j < jend) {
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
    const float alpha = exp2f(m_run - m_new);
    const float pj = j < jend ? exp2f(s - m_new) : 0.f;
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
    const int nkeys = (int)min((int64_t)128, jend - c0);
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
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < MAXD / 128; k++) {
    const int d = tid + 128 * k;
    if (d < D) Conv<T>::store(out, qoff + d, l_run > 0.f ? o[k] / l_run : 0.f);
  }
}

template <typename T, int BITS, int D, int GS>
int launch_decode(const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks, const void* kb,
                  const uint32_t* vp, const void* vs, const void* vb, Geometry geo, float scale, void* out,
                  hipStream_t s) {
  constexpr int TPW = D <= 128 ? 4 : 2;
  constexpr int MAXC = 128 * TPW;
  const int64_t span = geo.valid_len ? geo.cap : geo.n_kv;  // per-row upper bound on keys
  // aim for ~4 workgroups per CU over the whole launch
  const int64_t target = (int64_t)mlxq::device_cu_count() * 4;
  int64_t want = (span * B * Hkv + target - 1) / target;
  int chunk = 128;
  while (chunk < MAXC && chunk < want) chunk *= 2;
  const int64_t nchunks = span > 0 ? (span + chunk - 1) / chunk : 1;
  MLXQ_CHECK(nchunks < 65536, "kv length too large for one launch");
  uint32_t* counters = nullptr;
  void* pws = nullptr;
  const int nrep = Hq / Hkv;
  const size_t pbytes = (size_t)B * Hkv * nchunks * nrep * (D + 2) * sizeof(float);
  int rc = mlxq::workspace(pbytes, (size_t)B * Hkv, &counters, &pws, s);
  if (rc) return rc;
  dim3 grid((unsigned)nchunks, (unsigned)Hkv, (unsigned)B);
  hipLaunchKernelGGL((sdpa_decode_mfma_kernel<T, BITS, D, GS, TPW>), grid, dim3(256), 0, s, (const uint16_t*)q, kp,
                     (const uint16_t*)ks, (const uint16_t*)kb, vp, (const uint16_t*)vs, (const uint16_t*)vb, Hq,
                     Hkv, geo, scale, chunk, (uint16_t*)out, (float*)pws, counters);
  MLXQ_LAUNCHED("sdpa_decode_mfma_kernel");
  return MLXQ_OK;
}

template <typename T, int BITS>
int launch_decode_d(int D, int gs, const void* q, int B, int Hq, int Hkv, const uint32_t* kp, const void* ks,
                    const void* kb, const uint32_t* vp, const void* vs, const void* vb, Geometry geo, float scale,
                    void* out, hipStream_t s) {
#define DEC(DV, GV)                                                                                             \
  if (D == DV && gs == GV)                                                                                      \
    return launch_decode<T, BITS, DV, GV>(q, B, Hq, Hkv, kp, ks, kb, vp, vs, vb, geo, scale, out, s);
  DEC(128, 32) DEC(128, 64) DEC(128, 128)
  DEC(256, 32) DEC(256, 64) DEC(256, 128)
  if constexpr (BITS == 8) {
    DEC(64, 32) DEC(64, 64)
  }
#undef DEC
  return mlxq::fail(MLXQ_ERR_UNSUPPORTED, "decode: no MFMA instance for this head_dim/group_size");
}

bool decode_mfma_ok(int dtype, int bits, int D, int gs, int nrep) {
  if (!mlxq::is_half_dtype(dtype)) return false;
  if (bits != 4 && bits != 8) return false;
  const bool dok = D == 128 || D == 256 || (bits == 8 && D == 64 && gs <= 64);
  if (!dok) return false;
  return nrep * (D / gs) <= 16;
}

}  // namespace

extern "C" int mlxq_quantized_sdpa(const void* q, int dtype, int B, int Hq, int Hkv, int Lq, int D,
                                   const uint32_t* k_packed, const void* k_scales, const void* k_biases,
                                   const uint32_t* v_packed, const void* v_scales, const void* v_biases,
                                   int64_t kv_capacity, int64_t n_kv, const int32_t* valid_len,
                                   const int32_t* ring_offset, int mask_mode, int window, float scale,
                                   int group_size, int bits, void* out, void* stream) {
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
  MLXQ_CHECK(mask_mode == MLXQ_MASK_NONE || mask_mode == MLXQ_MASK_CAUSAL, "unknown mask mode");
  MLXQ_CHECK(window >= 0, "negative window");
  if (B == 0 || Hq == 0 || Lq == 0) return MLXQ_OK;
  MLXQ_CHECK(q && k_packed && k_scales && k_biases && v_packed && v_scales && v_biases && out, "null buffer");
  MLXQ_CHECK((uintptr_t)q % 16 == 0 && (uintptr_t)k_packed % 16 == 0 && (uintptr_t)v_packed % 16 == 0,
             "q and packed caches must be 16-byte aligned");
  hipStream_t s = mlxq::resolve_stream(stream);
  Geometry geo{kv_capacity, valid_len ? kv_capacity : n_kv, valid_len, ring_offset};
  const int nrep = Hq / Hkv;
  // Lq = 1 attends every valid key under either mask (its position is the last one)
  const bool decode = Lq == 1 && (mask_mode == MLXQ_MASK_NONE || window == 0);
  if (decode && decode_mfma_ok(dtype, bits, D, group_size, nrep)) {
    if (dtype == MLXQ_BFLOAT16)
      return bits == 4 ? launch_decode_d<BF16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                  v_packed, v_scales, v_biases, geo, scale, out, s)
                       : launch_decode_d<BF16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases,
                                                  v_packed, v_scales, v_biases, geo, scale, out, s);
    return bits == 4 ? launch_decode_d<F16, 4>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases, v_packed,
                                               v_scales, v_biases, geo, scale, out, s)
                     : launch_decode_d<F16, 8>(D, group_size, q, B, Hq, Hkv, k_packed, k_scales, k_biases, v_packed,
                                               v_scales, v_biases, geo, scale, out, s);
  }
  const int causal = mask_mode == MLXQ_MASK_CAUSAL;
  dim3 grid((unsigned)Lq, (unsigned)Hq, (unsigned)B);
  MLXQ_DISPATCH_T(dtype, TT, {
    switch (bits) {
      case 2:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 2>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out);
        break;
      case 4:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 4>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out);
        break;
      default:
        hipLaunchKernelGGL((sdpa_generic_kernel<TT, 8>), grid, dim3(128), 0, s, q, k_packed, k_scales, k_biases,
                           v_packed, v_scales, v_biases, Hq, Hkv, Lq, D, group_size, geo, causal, window, scale, out);
        break;
    }
  });
  MLXQ_LAUNCHED("sdpa_generic_kernel");
  return MLXQ_OK;
}
