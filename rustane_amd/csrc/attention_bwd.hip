// Fused causal attention backward (kernels/sdpa_bwd.rs:46-161), flash style:
//   P = softmax(Q K^T scale) is recomputed from the forward's per-query
//   log-sum-exp, dP = dO V^T, D = rowsum(P * dP), dS = P (dP - D) scale,
//   dQ = dS K, dK = dS^T Q, dV = P^T dO,
// with every score block kept in registers: nothing of size S^2 goes to
// memory. The arithmetic per element is the unfused path's (fp32 scores and
// dP, P and dS rounded to fp16 as MFMA operands, D summed in fp32 from the
// unrounded P and dP), in a different summation order.
//
// Both kernels use the forward kernel's 32x32x16 MFMA layouts (attention.hip):
// a row tile [32][hd] is read as A-operand rows in swap23 slot order (chunk c
// of row r at r*NCH + (c ^ (swap23(r) % NCH))), so the 8 accumulator
// registers 8j..8j+7 of lane half h2 hold the consecutive rows 16j+8h2..+7
// and serve directly as a B operand; a column tile [hd][32] (chunk c of row e
// at e*4 + (c ^ ((e >> 2) & 3))) gives A fragments of one hd row and 8
// consecutive keys or queries.
//
// attn_bwd_dq_kernel, per (PQ query blocks, head, sequence), PQ x PK waves
// (PK key parts): S^T = K Q^T and dP^T = V dO^T per key block, two passes
// over the keys (D first, then dQ^T += K^T dS^T); with two key halves
// (PQ = 2, as the forward) the halves add their D and dQ through LDS.
//
// attn_bwd_dkv_kernel, per (PB key blocks, sequence and KV head), PB x PH
// waves (PH query parts): the wave's K and V rows stay in registers
// as B operands, S = Q K^T and dP = dO V^T per query block of every head of
// the group (the GQA sum over heads is the loop), dV^T += dO^T P and
// dK^T += Q^T dS; with two query halves (PB = 2) the halves add their
// partials through LDS.
#include "internal.hpp"

namespace hb {

namespace {

// dQKV row and transpose of 4 consecutive features f0..f0+3 of token
// (b, s), column col. Q and K gradients go through the inverse of the
// forward's RoPE rotation at position s (layer.rs:1880-1897
// rope_backward_inplace): dx[2i] = d[2i] c + d[2i+1] s, dx[2i+1] = d[2i+1] c
// - d[2i] s.
HB_DEV void store_grad4(const AttnBwd& p, int b, int s, int col, int f0, f32x4 v, bool rope) {
  f32x4 o = v;
  if (rope) {
    const float4 r = p.rope[(size_t)(f0 >> 2) * p.rope_ld + s];  // f0 % 4 == 0
    const float2 c0 = make_float2(r.x, r.y), c1 = make_float2(r.z, r.w);
    o.x = v.x * c0.x + v.y * c0.y;
    o.y = v.y * c0.x - v.x * c0.y;
    o.z = v.z * c1.x + v.w * c1.y;
    o.w = v.w * c1.x - v.z * c1.y;
  }
  f16x4 h;
  h.x = (f16)o.x;
  h.y = (f16)o.y;
  h.z = (f16)o.z;
  h.w = (f16)o.w;
  const int tok = b * p.S + s;
  *(f16x4*)(p.dqkv + (size_t)tok * p.ld + col) = h;
  p.dqkvT[(size_t)col * p.tld + tok] = h.x;
  p.dqkvT[(size_t)(col + 1) * p.tld + tok] = h.y;
  p.dqkvT[(size_t)(col + 2) * p.tld + tok] = h.z;
  p.dqkvT[(size_t)(col + 3) * p.tld + tok] = h.w;
}

template <int HD>
HB_DEV int row_chunk(int r, int c) {  // row tile: chunk c of row r
  constexpr int NCH = HD / 8;
  return r * NCH + (c ^ (swap23(r) % NCH));
}
HB_DEV int col_chunk(int e, int c) { return e * 4 + (c ^ ((e >> 2) & 3)); }  // column tile

}  // namespace

template <int HD, int PQ, int PK>
__global__ __launch_bounds__(PQ * PK * 64, 1) void attn_bwd_dq_kernel(AttnBwd p) {
  constexpr int PW = PQ * PK;  // waves: query blocks x key parts
  constexpr int KS = HD / 16, MB = HD / 32, NCH = HD / 8, KT8 = 4 * HD;
  constexpr int NKIND = 3;  // K rows, V rows, K^T columns
  constexpr int NLD = NKIND * PK * KT8 / (PW * 64);
  static_assert(NLD * PW * 64 == NKIND * PK * KT8, "loader coverage");
  // two tile buffers: iteration n computes from buffer n & 1 while the tiles
  // of n + 1 go into the other one (one barrier per iteration)
  constexpr int NTILE = NKIND * PK * KT8, NMERGE = PK == 2 ? PQ * MB * 16 * 64 * 4 / 16 : 0;
  __shared__ f16x8 s_t[2 * NTILE > NMERGE ? 2 * NTILE : NMERGE];
  __shared__ float s_d[PQ][64];

  const int tid = threadIdx.x, lane = tid & 63, h2 = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int qs = wave % PQ, kh = wave / PQ;
  const int nqb = (p.S + 31) / 32, ngr = (nqb + PQ - 1) / PQ;
  const int gr = ngr - 1 - blockIdx.x;  // heaviest groups first
  // query blocks gr, gr + ngr, ... (as in the forward kernel: groups of
  // nearly equal causal work)
  const int qb = gr + ngr * qs;
  const bool active = qb < nqb;
  const int nkb = gr + ngr * min(PQ - 1, (nqb - 1 - gr) / ngr) + 1;
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (p.H / p.KVH), z = b * p.KVH + kvh;
  const int qi = qb * 32 + li;
  const bool qok = active && qi < p.S;
  const size_t qrow = ((size_t)b * p.H + h) * p.Sp;

  f16x8 qf[KS], df[KS];
  float L2 = 0.f;
  if (active) {
    const size_t qo = (qrow + qi) * HD + 8 * h2;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      qf[j] = *(const f16x8*)(p.q + qo + 16 * j);
      df[j] = *(const f16x8*)(p.dO + qo + 16 * j);
    }
    if (qi < p.S) L2 = p.lse[qrow + qi];
  }

  const f16* kz = p.k + (size_t)z * p.Sp * HD;
  const f16* vz = p.v + (size_t)z * p.Sp * HD;
  const f16* ktz = p.kT + (size_t)z * HD * p.Sp;
  f16x8 reg[NLD];
  auto gload = [&](int n, bool with_t) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int x = i * PW * 64 + tid, tile = x / KT8, y = x % KT8;
      const int kind = tile / PK, kb = min(n * PK + tile % PK, nkb - 1);
      if (kind < 2) {
        const f16* base = kind == 0 ? kz : vz;
        reg[i] = *(const f16x8*)(base + ((size_t)kb * 32 + y / NCH) * HD + (y % NCH) * 8);
      } else if (with_t) {
        reg[i] = *(const f16x8*)(ktz + (size_t)(y >> 2) * p.Sp + kb * 32 + (y & 3) * 8);
      }
    }
  };
  auto lstore = [&](int buf, bool with_t) {
    f16x8* st = s_t + buf * NTILE;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int x = i * PW * 64 + tid, tile = x / KT8, y = x % KT8;
      if (tile / PK < 2)
        st[tile * KT8 + row_chunk<HD>(y / NCH, y % NCH)] = reg[i];
      else if (with_t)
        st[tile * KT8 + col_chunk(y >> 2, y & 3)] = reg[i];
    }
  };

  const float sl2 = p.scale * HB_LOG2E;
  const int krow = swap23(li);
  const int niter = (nkb + PK - 1) / PK;
  // the key loop of one pass: body(n, tile buffer) on every iteration's tiles
  auto keyloop = [&](bool with_t, auto&& body) {
    gload(0, with_t);
    lstore(0, with_t);
    if (niter > 1) gload(1, with_t);
    lds_barrier();
    for (int n = 0; n < niter; ++n) {
      body(n, s_t + (n & 1) * NTILE);
      if (n + 1 < niter) {
        lstore((n + 1) & 1, with_t);  // that buffer was last read in iteration n - 1
        if (n + 2 < niter) gload(n + 2, with_t);
      }
      lds_barrier();
    }
  };
  // S^T and dP^T of key block kb against this wave's queries; s becomes P
  auto block = [&](const f16x8* st, int kb, f32x16& s, f32x16& dp) {
    const f16x8* sk = st + kh * KT8;
    const f16x8* sv = st + (PK + kh) * KT8;
    s = f32x16{};
    dp = f32x16{};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int ko = krow * NCH + ((2 * j + h2) ^ (li % NCH));
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(sk[ko], qf[j], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(sv[ko], df[j], dp, 0, 0, 0);
    }
    // masked entries get exp2(-inf) = 0: a select on the argument, no branch
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb * 32 + swap23(8 * (r >> 2) + 4 * h2 + (r & 3));
      s[r] = exp2f((qok && key <= qi) ? s[r] * sl2 - L2 : -INFINITY);
    }
  };

  // pass 1: D = rowsum(P * dP) over this wave's key half, then over both
  float dsum = 0.f;
  keyloop(false, [&](int n, const f16x8* st) {
    const int kb = n * PK + kh;
    if (!active || kb > qb) return;  // wave-uniform
    f32x16 s, dp;
    block(st, kb, s, dp);
#pragma unroll
    for (int r = 0; r < 16; ++r) dsum += s[r] * dp[r];
  });
  dsum += __shfl_xor(dsum, 32, 64);  // both lanes of a query pair
  float D = dsum;
  if constexpr (PK == 2) {
    if (kh == 1) s_d[qs][lane] = dsum;
    lds_barrier();
    const float Dq = kh == 0 ? dsum + s_d[qs][lane] : 0.f;
    lds_barrier();
    if (kh == 0) s_d[qs][lane] = Dq;
    lds_barrier();
    D = s_d[qs][lane];
  }
  if (kh == 0 && qok && h2 == 0) p.D[qrow + qi] = D;

  // pass 2: dS^T = P (dP - D) scale, dQ^T += K^T dS^T
  f32x16 o[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) o[m] = f32x16{};
  keyloop(true, [&](int n, const f16x8* st) {
    const int kb = n * PK + kh;
    if (!active || kb > qb) return;
    f32x16 s, dp;
    block(st, kb, s, dp);
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = s[r] * (dp[r] - D) * p.scale;
    const f16x8* skt = st + (2 * PK + kh) * KT8;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f16x8 db;
#pragma unroll
      for (int i = 0; i < 8; ++i) db[i] = (f16)s[8 * j + i];
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const int e = m * 32 + li;
        o[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(skt[col_chunk(e, 2 * j + h2)], db, o[m], 0, 0, 0);
      }
    }
  });

  // with two key halves, half 1 hands its dQ^T to half 0 (same lane, same
  // slots); the key loop ended on a barrier, so the tile buffers are free
  if constexpr (PK == 2) {
    float* s_o = (float*)s_t + qs * (MB * 16 * 64);
    if (kh == 1) {
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_o[(m * 16 + r) * 64 + lane] = o[m][r];
    }
    lds_barrier();
    if (kh == 1) return;
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[m][r] += s_o[(m * 16 + r) * 64 + lane];
  }
  if (!qok) return;
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int f0 = m * 32 + 8 * g + 4 * h2;
      f32x4 v;
      v.x = o[m][4 * g + 0];
      v.y = o[m][4 * g + 1];
      v.z = o[m][4 * g + 2];
      v.w = o[m][4 * g + 3];
      store_grad4(p, b, qi, h * HD + f0, f0, v, true);
    }
}

template <int HD, int PB, int PH>
__global__ __launch_bounds__(PB * PH * 64, 1) void attn_bwd_dkv_kernel(AttnBwd p) {
  constexpr int PW = PB * PH;  // waves: key blocks x query parts
  constexpr int KS = HD / 16, MB = HD / 32, NCH = HD / 8, KT8 = 4 * HD;
  constexpr int NKIND = 4;  // Q rows, dO rows, Q^T columns, dO^T columns
  constexpr int NLD = NKIND * PH * KT8 / (PW * 64);
  static_assert(NLD * PW * 64 == NKIND * PH * KT8, "loader coverage");
  // two tile buffers (one barrier per iteration, as in the dQ kernel)
  constexpr int NTILE = NKIND * PH * KT8, NMERGE = PH == 2 ? PB * 2 * MB * 16 * 64 * 4 / 16 : 0;
  __shared__ f16x8 s_t[2 * NTILE > NMERGE ? 2 * NTILE : NMERGE];
  __shared__ float s_ld[2][PH][2][32];  // log-sum-exp and D of the iteration's query blocks

  const int tid = threadIdx.x, lane = tid & 63, h2 = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kbi = wave % PB, qh = wave / PB;
  const int nb = (p.S + 31) / 32;  // key blocks = query blocks
  const int grp = blockIdx.x;      // group 0 sees the most query blocks: launched first
  // key blocks grp, grp + ngr, ...: every group spans the sequence, so the
  // groups' causal work is nearly equal
  const int ngr = (nb + PB - 1) / PB;
  const int kb = grp + ngr * kbi;
  const bool active = kb < nb;
  const int z = blockIdx.y, b = z / p.KVH, g = z - b * p.KVH;
  const int rep = p.H / p.KVH;
  const int ki = kb * 32 + li;
  const int qstart = grp;              // first query block that sees the group's keys
  const int nq = nb - qstart;           // query blocks per head
  const int npairs = rep * nq;          // (head, query block) pairs
  const int niter = (npairs + PH - 1) / PH;

  f16x8 kf[KS], vf[KS];
  if (active) {
    const size_t ko = ((size_t)z * p.Sp + ki) * HD + 8 * h2;
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      kf[j] = *(const f16x8*)(p.k + ko + 16 * j);
      vf[j] = *(const f16x8*)(p.v + ko + 16 * j);
    }
  }

  const size_t rq = (size_t)rep * p.Sp;
  f16x8 reg[NLD];
  float aux = 0.f;
  auto pair_of = [&](int n, int hq, int& r, int& qb) {
    const int pi = min(n * PH + hq, npairs - 1);
    r = pi / nq;
    qb = qstart + (pi - r * nq);
  };
  auto gload = [&](int n) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int x = i * PW * 64 + tid, tile = x / KT8, y = x % KT8;
      const int kind = tile / PH;
      int r, qb;
      pair_of(n, tile % PH, r, qb);
      if (kind < 2) {
        const f16* base = kind == 0 ? p.q : p.dO;
        const size_t row = ((size_t)b * p.H + g * rep + r) * p.Sp + qb * 32 + y / NCH;
        reg[i] = *(const f16x8*)(base + row * HD + (y % NCH) * 8);
      } else {
        const f16* base = (kind == 2 ? p.qT : p.dOT) + (size_t)z * HD * rq;
        reg[i] = *(const f16x8*)(base + (size_t)(y >> 2) * rq + (size_t)r * p.Sp + qb * 32 + (y & 3) * 8);
      }
    }
    if (tid < PH * 2 * 32) {  // thread: (query half, lse or D, query)
      const int hq = tid / 64, which = (tid >> 5) & 1, qq = tid & 31;
      int r, qb;
      pair_of(n, hq, r, qb);
      const int qpos = qb * 32 + qq;
      const size_t idx = ((size_t)b * p.H + g * rep + r) * p.Sp + qpos;
      aux = qpos < p.S ? (which ? p.D[idx] : p.lse[idx]) : 0.f;
    }
  };
  auto lstore = [&](int buf) {
    f16x8* st = s_t + buf * NTILE;
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int x = i * PW * 64 + tid, tile = x / KT8, y = x % KT8;
      if (tile / PH < 2)
        st[tile * KT8 + row_chunk<HD>(y / NCH, y % NCH)] = reg[i];
      else
        st[tile * KT8 + col_chunk(y >> 2, y & 3)] = reg[i];
    }
    if (tid < PH * 2 * 32) s_ld[buf][tid / 64][(tid >> 5) & 1][tid & 31] = aux;
  };

  const float sl2 = p.scale * HB_LOG2E;
  const int qrow = swap23(li);
  f32x16 dk[MB], dv[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    dk[m] = f32x16{};
    dv[m] = f32x16{};
  }
  auto body = [&](int n, int buf) {
    if (!active || n * PH + qh >= npairs) return;  // wave-uniform
    int r, qb;
    pair_of(n, qh, r, qb);
    if (qb < kb) return;  // every query of the block precedes every key
    const f16x8* st = s_t + buf * NTILE;
    const f16x8* sq = st + (0 * PH + qh) * KT8;
    const f16x8* sd = st + (1 * PH + qh) * KT8;
    const f16x8* sqt = st + (2 * PH + qh) * KT8;
    const f16x8* sdt = st + (3 * PH + qh) * KT8;
    f32x16 s = {}, dp = {};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      const int qo = qrow * NCH + ((2 * j + h2) ^ (li % NCH));
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(sq[qo], kf[j], s, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_f16(sd[qo], vf[j], dp, 0, 0, 0);
    }
    // rows are the queries qb*32 + swap23(slot), columns this lane's key ki;
    // their log-sum-exp and D are read from LDS together, then masked
    // entries get exp2(-inf) = 0 (a select on the argument, no branch)
    float lq[16], dq[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int qq = swap23(8 * (e >> 2) + 4 * h2 + (e & 3));
      lq[e] = s_ld[buf][qh][0][qq];
      dq[e] = s_ld[buf][qh][1][qq];
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int qpos = qb * 32 + swap23(8 * (e >> 2) + 4 * h2 + (e & 3));
      const float pe = exp2f((ki <= qpos && qpos < p.S) ? s[e] * sl2 - lq[e] : -INFINITY);
      s[e] = pe;
      dp[e] = pe * (dp[e] - dq[e]) * p.scale;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f16x8 pb, db;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pb[i] = (f16)s[8 * j + i];
        db[i] = (f16)dp[8 * j + i];
      }
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const int c = col_chunk(m * 32 + li, 2 * j + h2);
        dv[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sdt[c], pb, dv[m], 0, 0, 0);
        dk[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(sqt[c], db, dk[m], 0, 0, 0);
      }
    }
  };
  gload(0);
  lstore(0);
  if (niter > 1) gload(1);
  lds_barrier();
  for (int n = 0; n < niter; ++n) {
    body(n, n & 1);
    if (n + 1 < niter) {
      lstore((n + 1) & 1);  // that buffer was last read in iteration n - 1
      if (n + 2 < niter) gload(n + 2);
    }
    lds_barrier();
  }

  // with two query halves, half 1 hands its dK^T and dV^T to half 0 of the
  // same key block (the loop ended on a barrier: the tile buffers are free)
  if constexpr (PH == 2) {
    float* s_o = (float*)s_t + kbi * (2 * MB * 16 * 64);
    if (qh == 1) {
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          s_o[(m * 16 + e) * 64 + lane] = dk[m][e];
          s_o[((MB + m) * 16 + e) * 64 + lane] = dv[m][e];
        }
    }
    lds_barrier();
    if (qh == 1) return;
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        dk[m][e] += s_o[(m * 16 + e) * 64 + lane];
        dv[m][e] += s_o[((MB + m) * 16 + e) * 64 + lane];
      }
  }
  if (!active || ki >= p.S) return;
  const int colk = p.q_dim + g * HD, colv = p.q_dim + p.kv_dim + g * HD;
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int f0 = m * 32 + 8 * q4 + 4 * h2;
      f32x4 a, c;
      a.x = dk[m][4 * q4 + 0];
      a.y = dk[m][4 * q4 + 1];
      a.z = dk[m][4 * q4 + 2];
      a.w = dk[m][4 * q4 + 3];
      c.x = dv[m][4 * q4 + 0];
      c.y = dv[m][4 * q4 + 1];
      c.z = dv[m][4 * q4 + 2];
      c.w = dv[m][4 * q4 + 3];
      store_grad4(p, b, ki, colk + f0, f0, a, true);
      store_grad4(p, b, ki, colv + f0, f0, c, false);
    }
}

namespace {
// Four query blocks (dQ) or four key blocks (dK/dV) per workgroup share each
// staged tile once that still leaves two workgroups per CU (7B, one sequence
// of 2048: forward + backward 136.1 -> 129.5 ms; 8 query blocks for dQ:
// 125.0 -> 119.9 ms); otherwise two blocks, with the key or query range split
// in halves.
constexpr long HB_BWD_WIDE_MIN = 512;
template <int HD>
void launch_bwd(const AttnBwd& p, hipStream_t st) {
  const int nb = (p.S + 31) / 32;
  const long hb = (long)p.H * p.B, zb = (long)p.KVH * p.B;
  // dQ: 8 query blocks per workgroup (8 waves, hd = 128 only: one K, V and
  // K^T tile set covers 512 threads' loads) while that still gives every CU
  // one workgroup, else 4 with two workgroups per CU, else 2 with the key
  // range split in halves. dK/dV: 4 key blocks, else 2 with the query range
  // split (8 waves would need the K and V rows out of registers: the wave's
  // dK, dV, K and V already fill 224 of its 256 registers)
  bool dq8 = false;
  if constexpr (HD == 128) {
    if ((long)((nb + 7) / 8) * hb >= HB_BWD_WIDE_MIN / 2) {
      hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, 8, 1>), dim3((nb + 7) / 8, p.H, p.B), dim3(512), 0, st, p);
      dq8 = true;
    }
  }
  if (dq8) {
  } else if ((long)((nb + 3) / 4) * hb >= HB_BWD_WIDE_MIN)
    hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, 4, 1>), dim3((nb + 3) / 4, p.H, p.B), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((attn_bwd_dq_kernel<HD, 2, 2>), dim3((nb + 1) / 2, p.H, p.B), dim3(256), 0, st, p);
  if ((long)((nb + 3) / 4) * zb >= HB_BWD_WIDE_MIN)
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<HD, 4, 1>), dim3((nb + 3) / 4, p.B * p.KVH), dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<HD, 2, 2>), dim3((nb + 1) / 2, p.B * p.KVH), dim3(256), 0, st, p);
}
}  // namespace

hipError_t attention_backward_fused(const AttnBwd& p, hipStream_t st) {
  if (p.S < 1 || p.Sp < p.S || p.Sp % 32 || p.H % p.KVH || (p.hd != 64 && p.hd != 128) || !p.lse || !p.D)
    return hipErrorInvalidValue;
  if (p.hd == 128)
    launch_bwd<128>(p, st);
  else
    launch_bwd<64>(p, st);
  return hipGetLastError();
}

}  // namespace hb
