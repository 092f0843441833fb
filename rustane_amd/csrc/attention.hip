// Causal attention (kernels/sdpa_fwd.rs:132-149):
//   sc[s,t] = (Q'[s]·K'[t]) / sqrt(hd) + (t > s ? -65504 : 0); P = softmax_t(sc);
//   A[s] = sum_t P[s,t] V[t].
// The reference's additive -65504 underflows to exactly 0 after exp (every row
// keeps its diagonal term), so masked keys are skipped instead of added.
#include "internal.hpp"

namespace hb {

// ---- prefill: one workgroup of 4 waves per (64 queries, head, sequence) ---------
// S^T = K · Q^T on v_mfma_f32_32x32x16_f16 (rows = key slots, cols = queries):
// lane l owns query l%32 and the key slots 8*(r/4) + 4*(l/32) + r%4 of the
// 32-key block, so the online-softmax statistics of a query live in one lane
// pair (l, l^32). Key slot R holds key swap23(R) (bits 2 and 3 of the slot
// swapped), which makes the 8 score registers 8j..8j+7 of lane half h the
// consecutive keys 16j+8h .. 16j+8h+7. O^T = V^T · P^T then reuses those
// registers as the B operand, and the A operand (V^T row, the same 8 keys) is
// one 16-byte read.
//
// Wave w = qs + PQ*kh owns query block qs (of PQ) of the workgroup and the
// key blocks kb with kb % PK == kh (PK = 2): iteration n loads key blocks
// PK*n .. PK*n+PK-1 (K [32][hd] and V^T [hd][32] each) into LDS once, with
// 16-byte, wave-contiguous loads issued one iteration ahead, and every block
// is used by the PQ waves of its key half. Sharing a block between query
// blocks halves the bytes loaded per MFMA — a wave loading its own K/V needs
// ~128 B/clk per CU, four times what the L1-L2 path sustains — while splitting
// the key range over PK waves keeps the chain of dependent key blocks at half
// the row; the key halves merge through LDS at the end (the same rescaling an
// online softmax applies between blocks). Fragments are read from
// XOR-swizzled LDS without bank conflicts.
//
// PQ = 4 (8 waves) for long or many sequences: each key block then serves 128
// queries instead of 64, halving the L2 traffic per MFMA, once there are
// enough groups of 4 query blocks to give every CU two workgroups; short
// single sequences keep PQ = 2 (7B S = 512, B = 1: 256 workgroups). PQ = 8
// with PK = 1 (8 waves, each over the whole key range of its query block, no
// merge) once groups of 8 still give every CU one workgroup.


// SPLIT: Q, K, V and the probabilities in two-term fp16 form (common.hpp):
// each score and output product runs hi*hi + hi*lo + lo*hi MFMAs (the lo*lo
// term is below fp32 rounding of the sum), and the output rows are split rows.
template <int HD, bool SPLIT, int PQ, int PK>
__global__ __launch_bounds__(PQ * PK * 64, (SPLIT || PK == 1) ? 1 : 2) void attn_prefill_kernel(AttnPrefill p) {
  constexpr int PW = PQ * PK;          // waves
  constexpr int KS = HD / 16;          // k-steps over head dim
  constexpr int MB = HD / 32;          // 32-row blocks of O^T
  constexpr int NCH = HD / 8;          // 16-byte chunks per K row
  constexpr int KT8 = 4 * HD;          // 16-byte chunks per K tile (= per V^T tile)
  constexpr int NKIND = SPLIT ? 4 : 2;  // tile kinds: K, V^T (then their low parts)
  constexpr int NLD = NKIND * PK * KT8 / (PW * 64);  // 16-byte loads per thread per iteration
  static_assert(NLD * PW * 64 == NKIND * PK * KT8, "loader coverage");
  // K tiles (block kh: row r, chunk c at kh*KT8 + r*NCH + (c ^ (swap23(r) % NCH))), then
  // V^T tiles (block kh: row e, chunk c at (PK+kh)*KT8 + e*4 + (c ^ ((e >> 2) & 3))),
  // then (SPLIT) the same two for the low parts; after the loop the region
  // holds the key-half-1 waves' O for the merge
  constexpr int NTILE = NKIND * PK * KT8, NMERGE = PK == 2 ? PQ * MB * 16 * 64 * 4 / 16 : 0;
  __shared__ f16x8 s_kv[NTILE > NMERGE ? NTILE : NMERGE];
  __shared__ float s_ml[PQ][2][64];
  const int tid = threadIdx.x, lane = tid & 63, h2 = lane >> 5, li = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int qs = wave % PQ, kh = wave / PQ;
  const int nqb = (p.S + 31) / 32;
  const int ngr = (nqb + PQ - 1) / PQ;
  // Workgroups are dispatched round-robin over the 8 XCDs, each with its own
  // L2. The remap gives each XCD a contiguous range of (group, head,
  // sequence) in that order, so the groups that read one head's K and V run
  // on one XCD and that XCD's L2 fetches them once, instead of every XCD
  // fetching every head.
  const int nwg = gridDim.x * gridDim.y * gridDim.z;
  const int wg = xcd_remap(blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), nwg);
  const int gx = wg % gridDim.x, hy = (wg / gridDim.x) % gridDim.y, bz = wg / (gridDim.x * gridDim.y);
  const int gr = ngr - 1 - gx;  // heaviest groups first within a head
  // group gr holds the query blocks gr, gr + ngr, gr + 2 ngr, ...: every
  // group spans the sequence, so the groups' causal work is nearly equal
  // (contiguous groups left most CUs idle behind the last one); the
  // arithmetic of a query block does not depend on its group
  const int qb = gr + ngr * qs;  // >= nqb: this wave has no queries
  const bool active = qb < nqb;
  const int nkb = gr + ngr * min(PQ - 1, (nqb - 1 - gr) / ngr) + 1;  // key blocks the group needs
  const int h = hy, b = bz;
  const int kvh = h / (p.H / p.KVH);
  const int q0 = qb * 32;
  const int qi = q0 + li;

  f16x8 qf[KS], ql[SPLIT ? KS : 1];
  if (active) {
    const size_t qo = (((size_t)b * p.H + h) * p.q_rows + q0 + li) * HD + 8 * h2;
#pragma unroll
    for (int j = 0; j < KS; ++j) qf[j] = *(const f16x8*)(p.q + qo + 16 * j);
    if constexpr (SPLIT) {
#pragma unroll
      for (int j = 0; j < KS; ++j) ql[j] = *(const f16x8*)(p.q_lo + qo + 16 * j);
    }
  }

  const size_t koff = b * p.k_bstride + kvh * p.k_hstride;
  const size_t voff = ((size_t)b * p.KVH + kvh) * HD * p.vt_ld;
  const float sl2 = p.scale * HB_LOG2E;

  // thread tid, load i covers 16-byte chunk x = i*NT + tid (NT = PW*64) of the
  // iteration's NKIND*PK tiles (K blocks, then V^T blocks, then their low
  // parts). NT and KT8 are powers of two, so x's tile is a constant of i, or
  // of i and the wave when NT > KT8: written that way, the branches on the
  // tile kind below are uniform (from tid alone the compiler made them
  // divergent, with a wait in each).
  constexpr int NT = PW * 64;
  auto tile_of = [&](int i) {
    if constexpr (NT <= KT8)
      return (i * NT) / KT8;
    else
      return i * (NT / KT8) + (wave * 64) / KT8;
  };
  auto y_of = [&](int i) {
    if constexpr (NT <= KT8)
      return (i * NT) % KT8 + tid;
    else
      return tid % KT8;
  };
  static_assert(NT <= KT8 ? KT8 % NT == 0 : NT % KT8 == 0, "tiles and threads nest");
  f16x8 kvreg[NLD];
  auto gload = [&](int n) {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int tile = tile_of(i), y = y_of(i);
      const int kind = tile / PK;  // 0 K, 1 V^T, 2 K low, 3 V^T low
      const int kb = min(n * PK + (tile % PK), nkb - 1);
      if ((kind & 1) == 0) {
        const f16* kbase = (kind ? p.k_lo : p.k) + koff;
        kvreg[i] = *(const f16x8*)(kbase + ((size_t)kb * 32 + y / NCH) * HD + (y % NCH) * 8);
      } else {
        const f16* vbase = (kind > 1 ? p.vt_lo : p.vt) + voff;
        const int e = y >> 2, c = y & 3;
        kvreg[i] = *(const f16x8*)(vbase + (size_t)e * p.vt_ld + kb * 32 + c * 8);
      }
    }
  };
  auto lstore = [&]() {
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int tile = tile_of(i), y = y_of(i);
      if (((tile / PK) & 1) == 0) {
        const int r = y / NCH, c = y % NCH;
        s_kv[tile * KT8 + r * NCH + (c ^ (swap23(r) % NCH))] = kvreg[i];
      } else {
        const int e = y >> 2, c = y & 3;
        s_kv[tile * KT8 + e * 4 + (c ^ ((e >> 2) & 3))] = kvreg[i];
      }
    }
  };
  const f16x8* sk = s_kv + kh * KT8;
  const f16x8* sv = s_kv + (PK + kh) * KT8;
  const f16x8* skl = s_kv + (2 * PK + kh) * KT8;  // SPLIT only
  const f16x8* svl = s_kv + (3 * PK + kh) * KT8;

  f32x16 o[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) o[m] = f32x16{};
  float mrun = -INFINITY, lrun = 0.f;

  const int krow = swap23(li);  // key held in this lane's slot
  const int niter = (nkb + PK - 1) / PK;
  gload(0);
  for (int n = 0; n < niter; ++n) {
    lds_barrier();  // every wave is done with the previous iteration's tiles
    lstore();
    lds_barrier();  // the tiles are in LDS
    if (n + 1 < niter) gload(n + 1);
    const int kb = n * PK + kh;
    if (!active || kb > qb) continue;  // wave-uniform

    // all of the block's K fragments are read before the score MFMAs, so
    // the LDS reads overlap instead of each waiting in front of its MFMA
    f32x16 s = {};
    f16x8 kf[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) kf[j] = sk[krow * NCH + ((2 * j + h2) ^ (li % NCH))];
#pragma unroll
    for (int j = 0; j < KS; ++j) {
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[j], qf[j], s, 0, 0, 0);
      if constexpr (SPLIT) {
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(kf[j], ql[j], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x16_f16(skl[krow * NCH + ((2 * j + h2) ^ (li % NCH))], qf[j], s, 0,
                                                   0, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, SPLIT ? 2 * KS : KS, 0);  // the K fragment reads,
    __builtin_amdgcn_sched_group_barrier(0x008, SPLIT ? 3 * KS : KS, 0);  // then the score MFMAs
    // (Folding the scale into each exponent as fma(s, sl2, -mrun) ran 3-4%
    // faster but moved the 7B seq-2048 top-1 agreement with the oracle from
    // 2042 to 2036 of 2048: the scaled scores are rounded first, as here.)
    float mloc = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] *= sl2;
    if (kb == qb) {  // diagonal block: keys after the query are masked
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (kb * 32 + swap23(8 * (r >> 2) + 4 * h2 + (r & 3)) > qi) s[r] = -INFINITY;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, s[r]);
    // the lane pair (l, l ^ 32), in registers (common.hpp)
    mloc = xor32_op(mloc, [](float x, float y) { return fmaxf(x, y); });
    // The reference max mrun is only raised when a score exceeds it by more
    // than 2^8 (log2 units): probabilities stay <= 256 (exact in fp16 to the
    // same relative precision) and the final 1/l cancels the common scale,
    // so O and l are only rescaled on such jumps (always on the first block).
    if (__builtin_amdgcn_ballot_w64(mloc > mrun + 8.f)) {
      const float mnew = fmaxf(mrun, mloc);
      const float corr = exp2f(mrun - mnew);
      lrun *= corr;
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[m][r] *= corr;
      mrun = mnew;
    }
    // v_exp_f32 itself: the arguments are <= 8, and a result below 2^-126
    // (where exp2f would return a denormal) is 0 once rounded to fp16 and
    // vanishes in the query's sum l (>= 1: the lane pair holds the key of
    // the maximum) -- the same output bits, without exp2f's denormal range
    // scaling (5 more instructions per probability)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = __builtin_amdgcn_exp2f(s[r] - mrun);
      s[r] = e;
      lrun += e;  // this lane's keys; the lane pair is summed after the loop
    }

#pragma unroll
    for (int j = 0; j < 2; ++j) {
      f16x8 pb, pl;
#pragma unroll
      for (int i = 0; i < 8; ++i) pb[i] = (f16)s[8 * j + i];
      if constexpr (SPLIT) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pl[i] = (f16)(s[8 * j + i] - (float)pb[i]);
      }
#pragma unroll
      for (int m = 0; m < MB; ++m) {
        const int e = m * 32 + li;
        const int vo = e * 4 + ((2 * j + h2) ^ ((e >> 2) & 3));
        const f16x8 va = sv[vo];
        o[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pb, o[m], 0, 0, 0);
        if constexpr (SPLIT) {
          o[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va, pl, o[m], 0, 0, 0);
          o[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(svl[vo], pb, o[m], 0, 0, 0);
        }
      }
    }
  }
  lrun += __shfl_xor(lrun, 32, 64);  // both lanes of a query pair share mrun

  // The key-half-1 waves hand (o, m, l) to the key-half-0 wave of the same
  // query block (a wave with no key block has m = -inf and weight 0). Lane l
  // of both waves holds the same (query, row) slots, so the exchange is one
  // float per lane per register.
  float M = mrun, L = lrun;
  if constexpr (PK == 2) {
    float* s_o = (float*)s_kv + qs * (MB * 16 * 64);  // [MB*16][64] per query block
    lds_barrier();  // every wave is done with the tiles
    if (kh == 1) {
#pragma unroll
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) s_o[(m * 16 + r) * 64 + lane] = o[m][r];
      s_ml[qs][0][lane] = mrun;
      s_ml[qs][1][lane] = lrun;
    }
    lds_barrier();
    if (kh == 1 || !active) return;
    const float mw = s_ml[qs][0][lane];
    M = fmaxf(mrun, mw);
    const float c0 = exp2f(mrun - M);  // key half 0 always holds block 0, so mrun is finite
    const float cw = mw == -INFINITY ? 0.f : exp2f(mw - M);
    L = lrun * c0 + cw * s_ml[qs][1][lane];
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[m][r] = o[m][r] * c0 + cw * s_o[(m * 16 + r) * 64 + lane];
  } else {
    if (!active) return;
  }

  if (p.lse && qi < p.S && h2 == 0) p.lse[((size_t)b * p.H + h) * p.q_rows + qi] = M + log2f(L);
  if (qi < p.S) {
    const float inv = 1.0f / L;
    f16* op = p.out + ((size_t)b * p.S + qi) * (SPLIT ? 2 * p.H * HD : p.H * HD) + h * HD;
    const size_t lo = SPLIT ? (size_t)p.H * HD : 0;  // split rows: [hi | lo]
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 w;
        w.x = o[m][4 * g + 0] * inv;
        w.y = o[m][4 * g + 1] * inv;
        w.z = o[m][4 * g + 2] * inv;
        w.w = o[m][4 * g + 3] * inv;
        store_f16x4(op + m * 32 + 8 * g + 4 * h2, w, lo);
      }
  }
}

namespace {
template <int PQ, int PK>
hipError_t launch_prefill(const AttnPrefill& p, hipStream_t st) {
  const int nqb = (p.S + 31) / 32;
  dim3 grid((nqb + PQ - 1) / PQ, p.H, p.B), block(PQ * PK * 64);
  const bool split = p.q_lo != nullptr;
  if (p.hd == 128 && split)
    hipLaunchKernelGGL((attn_prefill_kernel<128, true, PQ, PK>), grid, block, 0, st, p);
  else if (p.hd == 128)
    hipLaunchKernelGGL((attn_prefill_kernel<128, false, PQ, PK>), grid, block, 0, st, p);
  else if (p.hd == 64 && split)
    hipLaunchKernelGGL((attn_prefill_kernel<64, true, PQ, PK>), grid, block, 0, st, p);
  else if (p.hd == 64)
    hipLaunchKernelGGL((attn_prefill_kernel<64, false, PQ, PK>), grid, block, 0, st, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}
}  // namespace

hipError_t attention_prefill(const AttnPrefill& p, hipStream_t st) {
  if (p.q_lo != nullptr && (!p.k_lo || !p.vt_lo)) return hipErrorInvalidValue;
  // PQ = 8 (one workgroup per CU) or 4 (two) when the grid still fills the
  // GPU (measured on the 7B shape: seq 2048 forward at B = 1 33.2 ms with
  // PQ = 2, 32.75 with 4, 31.5 -> 31.2 with 8; seq 512 at B = 8 55.7 -> 55.2)
  const int nqb = (p.S + 31) / 32;
  const long hb = (long)p.H * p.B;
  if ((long)((nqb + 7) / 8) * hb >= 256) return launch_prefill<8, 1>(p, st);
  if ((long)((nqb + 3) / 4) * hb >= 512) return launch_prefill<4, 2>(p, st);
  return launch_prefill<2, 2>(p, st);
}

// ---- decode: split the context into chunks --------------------------------
// Grid (chunk, head, sequence), NW waves per chunk. hd/8 lanes share one key
// row (16-byte loads, non-temporal: the cache is streamed once per step and
// should not displace the activations from L2; B = 16 decode 6.31 -> 5.98 ms
// per step): one wave instruction reads KPW consecutive key rows
// (1 KB), and the NW waves' instructions together cover one stripe of
// NW * KPW keys; a block is NIT stripes (NW * 32 keys). Per block each lane
// issues all of its K and V loads before using any (V does not depend on the
// scores); each wave keeps its own online softmax state across the chunk's
// blocks, and the waves merge through LDS into one partial (max, sum,
// unnormalised output) per chunk -- or, when one chunk spans the whole
// context, straight into the normalised fp16 attention row.
//
// Chunks: n per (sequence, head), sized at every step from the position
// (attn_chunk_keys: keys 0..pos in n near-equal ranges), so each of the
// B x H x n workgroups streams the same share of the cache whatever the
// position, and the launch shape does not depend on it (one HIP graph
// replays every step). n is enough for about 256 workgroups (one per CU), at
// most one per 512 keys of capacity: 5 chunks per head on the 7B shape at
// B = 1 and 2304 keys, one at B >= 8 (no partials, no combine), where 8-wave
// workgroups let two run on a CU, their blocks interleaving (B = 16: 97.5
// against 99.3 us per layer with 16 waves, one workgroup per CU). At B = 1
// the kernel is not bound by its workgroup count: 8 chunks of ~270 keys
// (256 workgroups) take the same 11.0 us as 5, and the Wo prologue's combine
// of 8 partials costs 0.8 us more.
//
// With several chunks the partials are combined by the consumer -- the Wo
// GEMV prologue (gemv.hip) when B * chunks is small -- or by
// attn_combine_kernel below, which folds them in the same order with the
// same arithmetic, so both give the same attention output.
constexpr int DMIN_CHUNK = 512;  // fewest keys of ctx_max per chunk

AttnChunking attn_decode_chunking(int ctx_max, int B, int H) {
  const int bh = std::max(1, B * H);
  const int most = std::max(1, (ctx_max + DMIN_CHUNK - 1) / DMIN_CHUNK);
  const int n = std::max(1, std::min(most, 256 / bh));
  return AttnChunking{n, n == 1 && bh >= 256 ? 8 : 16};
}

// SPLIT: q, K and V come in two-term fp16 form (common.hpp) and are summed to
// fp32 as they are loaded (the arithmetic is fp32 throughout).
template <int HD, bool SPLIT, int NW>
__global__ __launch_bounds__(NW * 64) void attn_decode_kernel(AttnDecode p) {
  constexpr int NT = NW * 64;
  constexpr int LPK = HD / 8;       // lanes per key row
  constexpr int KPW = 64 / LPK;     // keys per wave instruction
  constexpr int STRIPE = NW * KPW;  // keys per instruction of all waves
  constexpr int NIT = 32 / KPW;     // instructions per block (32 keys per wave)
  constexpr int BLOCK = NIT * STRIPE;
  __shared__ float s_m[NW], s_l[NW];
  __shared__ float s_o[NW][HD];

  const int pos = *p.d_pos;
  const int cl = attn_chunk_keys(pos, gridDim.x);
  const int c0 = blockIdx.x * cl;
  if (c0 > pos) return;
  const int cend = min(c0 + cl, pos + 1);  // keys c0 .. cend-1
  const int h = blockIdx.y, b = blockIdx.z;
  const int kvh = h / (p.H / p.KVH);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane / LPK, j = lane % LPK;

  const size_t qo = ((size_t)b * p.H + h) * HD + 8 * j;
  const f16x8 qv = *(const f16x8*)(p.q + qo);
  float qf[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qf[i] = (float)qv[i];
  if constexpr (SPLIT) {
    const f16x8 ql = *(const f16x8*)(p.q_lo + qo);
#pragma unroll
    for (int i = 0; i < 8; ++i) qf[i] += (float)ql[i];
  }
  const size_t kvo = b * p.bstride + kvh * p.hstride + 8 * j;
  const f16* kb = p.k + kvo;
  const f16* vb = p.v + kvo;
  const float sl2 = p.scale * HB_LOG2E;

  // Online softmax state of this lane's keys (m is wave-uniform).
  float m = -INFINITY, l = 0.f, acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int b0 = c0; b0 < cend; b0 += BLOCK) {
    const int kbase = b0 + wave * KPW + g;  // key of instruction i: kbase + i * STRIPE
    constexpr int NL = SPLIT ? NIT : 1;
    f16x8 kr[NIT], krl[NL];
    const f16x8 zero8 = {};
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      const int kk = kbase + i * STRIPE;
      kr[i] = kk < cend ? __builtin_nontemporal_load((const f16x8*)(kb + (size_t)kk * HD)) : zero8;
      if constexpr (SPLIT)
        krl[i] = kk < cend ? __builtin_nontemporal_load((const f16x8*)(p.k_lo + kvo + (size_t)kk * HD)) : zero8;
    }
    // Without low parts the V loads go out with K's, before the scores. With
    // them they follow the scores, in two halves, so that K's registers are
    // free again and one half of V (hi and lo) is live at a time.
    constexpr int NV = SPLIT ? NIT / 2 : NIT;
    f16x8 vr[NV], vrl[SPLIT ? NV : 1];
    auto load_v = [&](int i0) {
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        const int kk = kbase + (i0 + i) * STRIPE;
        vr[i] = kk < cend ? __builtin_nontemporal_load((const f16x8*)(vb + (size_t)kk * HD)) : zero8;
        if constexpr (SPLIT)
          vrl[i] = kk < cend ? __builtin_nontemporal_load((const f16x8*)(p.v_lo + kvo + (size_t)kk * HD)) : zero8;
      }
    };
    if constexpr (!SPLIT) load_v(0);
    auto kval = [&](int i, int e) { return SPLIT ? (float)kr[i][e] + (float)krl[i % NL][e] : (float)kr[i][e]; };
    float sc[NIT];
#pragma unroll
    for (int i = 0; i < NIT; ++i) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d += qf[e] * kval(i, e);
      d = group_sum<LPK>(d);
      sc[i] = (kbase + i * STRIPE < cend) ? d * sl2 : -INFINITY;
    }
    // wave-wide max over this block's keys (lanes of a group hold equal scores)
    float mb = sc[0];
#pragma unroll
    for (int i = 1; i < NIT; ++i) mb = fmaxf(mb, sc[i]);
    mb = fold_groups<LPK>(mb, [](float a, float c) { return fmaxf(a, c); });
    const float mn = fmaxf(m, mb);
    if (mn != -INFINITY) {
      if (m != mn) {  // rescale what earlier blocks left (nothing on the first)
        const float r = exp2f(m - mn);
        l *= r;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] *= r;
        m = mn;
      }
#pragma unroll
      for (int i0 = 0; i0 < NIT; i0 += NV) {
        if constexpr (SPLIT) load_v(i0);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          // v_exp_f32 itself: pk <= 1, and a pk below 2^-126 (where exp2f
          // would return a denormal) vanishes once the lanes' sums meet the
          // maximum key's (pk = 1), so exp2f's denormal scaling changes no
          // result
          const float pk = __builtin_amdgcn_exp2f(sc[i0 + i] - m);
          l += pk;
#pragma unroll
          for (int e = 0; e < 8; ++e)
            acc[e] += pk * (SPLIT ? (float)vr[i][e] + (float)vrl[i % (SPLIT ? NV : 1)][e] : (float)vr[i][e]);
        }
      }
    }
  }
  {
    const auto add = [](float a, float c) { return a + c; };
    l = fold_groups<LPK>(l, add);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = fold_groups<LPK>(acc[e], add);
  }
  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
  if (g == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s_o[wave][8 * j + e] = acc[e];
  }
  __syncthreads();
  float M = s_m[0];
#pragma unroll
  for (int v = 1; v < NW; ++v) M = fmaxf(M, s_m[v]);
  // Wave weights exp2(m_w - M); a wave whose keys are all past the chunk has
  // m_w = -inf and weight 0.
  auto wt = [&](int v) { return s_m[v] == -INFINITY ? 0.f : exp2f(s_m[v] - M); };
  float L = 0.f;
#pragma unroll
  for (int v = 0; v < NW; ++v) L += wt(v) * s_l[v];
  const size_t head = (size_t)b * p.H + h;
  if (gridDim.x == 1) {
    // One chunk: the normalised attention row, fp16 (split rows [B][2*H*hd]
    // hi | lo with two-term inputs), as attention_combine would write it.
    const float iL = 1.0f / L;
    for (int e = tid; e < HD; e += NT) {
      float o = 0.f;
#pragma unroll
      for (int v = 0; v < NW; ++v) o += wt(v) * s_o[v][e];
      o *= iL;
      const f16 hi = (f16)o;
      if (p.q_lo) {
        f16* op = p.out + (size_t)b * 2 * p.H * HD + h * HD + e;
        op[0] = hi;
        op[(size_t)p.H * HD] = (f16)(o - (float)hi);
      } else if (p.out_frag) {  // the Wo GEMV's B-fragment order over K = H*hd
        const int k = h * HD + e;
        p.out[((size_t)(k >> 5) * 64 + b + 16 * ((k & 31) >> 3)) * 8 + (k & 7)] = hi;
      } else {
        p.out[head * HD + e] = hi;
      }
    }
    return;
  }
  const size_t slot = head * gridDim.x + blockIdx.x;
  for (int e = tid; e < HD; e += NT) {
    float o = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) o += wt(v) * s_o[v][e];
    p.part_o[slot * HD + e] = o;
  }
  if (tid == 0) {
    p.part_ml[slot * 2] = M;
    p.part_ml[slot * 2 + 1] = L;
  }
}

// out[b][h*hd + e] from the chunk partials of (b, h): one thread per 8
// consecutive elements; max over the valid chunks, then weights exp2(m_c - M)
// in chunk order (the Wo GEMV prologue's combine, stage_attn in gemv.hip).
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnDecode p, int nch) {
  constexpr int GPH = HD / 8;
  const int gid = blockIdx.x * 256 + threadIdx.x;
  if (gid >= p.B * p.H * GPH) return;
  const int nvalid = attn_chunks_valid(*p.d_pos, nch);
  const int bh = gid / GPH, e0 = (gid % GPH) * 8;
  const float* pml = p.part_ml + (size_t)bh * nch * 2;
  const float* po = p.part_o + (size_t)bh * nch * HD + e0;
  float M = -INFINITY;
  for (int c = 0; c < nvalid; ++c) M = fmaxf(M, pml[2 * c]);
  float L = 0.f;
  f32x4 O0 = {}, O1 = {};
  for (int c = 0; c < nvalid; ++c) {
    const float w = exp2f(pml[2 * c] - M);
    L += w * pml[2 * c + 1];
    O0 += w * *(const f32x4*)(po + (size_t)c * HD);
    O1 += w * *(const f32x4*)(po + (size_t)c * HD + 4);
  }
  const float iL = 1.0f / L;
  if (p.q_lo) {  // split rows [B][2*H*hd]: hi | lo
    const int b = bh / p.H, h = bh - b * p.H;
    f16* op = p.out + (size_t)b * 2 * p.H * HD + h * HD + e0;
    store_f16x4(op, O0 * iL, (size_t)p.H * HD);
    store_f16x4(op + 4, O1 * iL, (size_t)p.H * HD);
    return;
  }
  f16x8 o;
  o[0] = (f16)(O0.x * iL);
  o[1] = (f16)(O0.y * iL);
  o[2] = (f16)(O0.z * iL);
  o[3] = (f16)(O0.w * iL);
  o[4] = (f16)(O1.x * iL);
  o[5] = (f16)(O1.y * iL);
  o[6] = (f16)(O1.z * iL);
  o[7] = (f16)(O1.w * iL);
  *(f16x8*)(p.out + (size_t)bh * HD + e0) = o;
}

namespace {
template <int NW>
hipError_t launch_decode(const AttnDecode& p, dim3 grid, bool split, hipStream_t st) {
  const dim3 block(NW * 64);
  if (p.hd == 128 && split)
    hipLaunchKernelGGL((attn_decode_kernel<128, true, NW>), grid, block, 0, st, p);
  else if (p.hd == 128)
    hipLaunchKernelGGL((attn_decode_kernel<128, false, NW>), grid, block, 0, st, p);
  else if (p.hd == 64 && split)
    hipLaunchKernelGGL((attn_decode_kernel<64, true, NW>), grid, block, 0, st, p);
  else if (p.hd == 64)
    hipLaunchKernelGGL((attn_decode_kernel<64, false, NW>), grid, block, 0, st, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}
}  // namespace

hipError_t attention_decode(const AttnDecode& p, hipStream_t st) {
  const AttnChunking ch = attn_decode_chunking(p.ctx_max, p.B, p.H);
  if (p.nch != ch.n) return hipErrorInvalidValue;
  const dim3 grid(ch.n, p.H, p.B);
  const bool split = p.q_lo != nullptr;
  if (split && (!p.k_lo || !p.v_lo)) return hipErrorInvalidValue;
  if (p.out_frag && (ch.n != 1 || split || p.B > 16 || (p.H * p.hd) % 32)) return hipErrorInvalidValue;
  return ch.waves == 8 ? launch_decode<8>(p, grid, split, st) : launch_decode<16>(p, grid, split, st);
}

hipError_t attention_combine(const AttnDecode& p, hipStream_t st) {
  const AttnChunking ch = attn_decode_chunking(p.ctx_max, p.B, p.H);
  if (p.nch != ch.n || ch.n < 2) return hipErrorInvalidValue;
  const int nch = ch.n;
  const int n = p.B * p.H * (p.hd / 8);
  if (p.hd == 128)
    hipLaunchKernelGGL(attn_combine_kernel<128>, dim3((n + 255) / 256), dim3(256), 0, st, p, nch);
  else if (p.hd == 64)
    hipLaunchKernelGGL(attn_combine_kernel<64>, dim3((n + 255) / 256), dim3(256), 0, st, p, nch);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace hb
