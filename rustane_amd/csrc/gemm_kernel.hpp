// Prefill GEMM kernel (launch policy in gemm_launch.hpp).
//
// C^T tile = W_tile · X_tile^T on v_mfma_f32_32x32x16_f16:
//   W [N, K] fp16, K contiguous (weights repacked output-major at upload)
//   X [T, K] fp16, K contiguous (token-major activations)
//   result(t, f) = sum_k X[t,k] * W[f,k], fp32 accumulate, handed to an epilogue.
// MFMA rows are output features and MFMA columns are tokens, so each lane ends
// up holding 4 consecutive features of one token — the shape every epilogue
// (RoPE pairs, SwiGLU pairs, residual float4) wants.
//
// LDS rows are 128 B (64 halfs) of eight 16-byte chunks; chunk c of row r is
// stored at c ^ swz(r), which keeps both the loaders' ds_write_b128 and the
// MFMA operands' ds_read_b128 free of bank conflicts for 32- and 64-bank LDS.
#pragma once
#include <type_traits>

#include "internal.hpp"

namespace hb {

HB_DEV int lds_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// f(integral_constant<int, I>) for I = B .. E-1, unrolled by the template
// expansion itself.
template <int B, int E, class F>
HB_DEV void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// Epilogues that read memory declare `Aux`, `Aux load(t, f0, fb)` and
// `operator()(t, f0, v, aux, fb)`, where fb is the wave-uniform start of the
// 32-feature block that holds f0; the others only `operator()(t, f0, v)`.
template <class E, class = void>
struct EpiAux {
  struct type {};
  static HB_DEV type load(const E&, int, int, int) { return {}; }
  static HB_DEV auto apply(const E& e, int t, int f0, f32x4 v, const type&, int) { return e(t, f0, v); }
};
template <class E>
struct EpiAux<E, std::void_t<typename E::Aux>> {
  using type = typename E::Aux;
  static HB_DEV type load(const E& e, int t, int f0, int fb) { return e.load(t, f0, fb); }
  static HB_DEV auto apply(const E& e, int t, int f0, f32x4 v, const type& a, int fb) {
    return e(t, f0, v, a, fb);
  }
};

// Epilogues with kStage copy a table the epilogue reads into the operand
// LDS once the main loop is done -- `stage<TT, NT>(lo, hi, t_base, f_base,
// tid)` by all threads, then `load_staged(lo, hi, t - t_base, TT, f0, fb)` in
// place of load() -- so that the epilogue's operand reads wait on LDS
// instead of behind its own global stores (one counter covers both).
template <class E, class = void>
struct EpiStage : std::false_type {};
template <class E>
struct EpiStage<E, std::void_t<decltype(E::kStage)>> : std::bool_constant<E::kStage> {};

// Epilogues with `Tok tok(t)`, `row(tok, fb)` and `store_row(row, f0, v, aux,
// fb)` can split their output addressing: tok() once per token of a lane, row()
// once per (32-feature block, token), store_row() per quad.
// Selected by `kRows`.
template <class E, class = void>
struct EpiRows : std::false_type {
  struct Tok {};
};
template <class E>
struct EpiRows<E, std::enable_if_t<E::kRows>> : std::true_type {
  using Tok = typename E::Tok;
};

// Epilogues with kSumSq return the sum of squares of the four values they
// stored; the kernel adds them up per workgroup and writes the total to
// epi.sq_out[tile] (one slot per output tile, fixed order for the reader).
template <class E, class = void>
struct EpiSumSq : std::false_type {};
template <class E>
struct EpiSumSq<E, std::void_t<decltype(E::kSumSq)>> : std::bool_constant<E::kSumSq> {};

// Pipeline: two 64-wide K slices are in flight in registers while the MFMAs
// consume a third from LDS. Iteration k computes slice k from LDS buffer k&1,
// issues the global loads of slice k+2 into register set k&1 and writes slice
// k+1 (register set (k+1)&1, loaded one iteration earlier) into LDS buffer
// (k+1)&1; one barrier per slice. The loop is unrolled by two so that both
// register sets have static names. Within an iteration sched_group_barrier
// fixes the order: LDS reads of k-step 0 first, then every MFMA is followed by
// one LDS read of the next k-step (k-steps 0..2), and the global loads are
// spread one per MFMA over k-steps 0..2 while the LDS writes are spread over
// k-steps WSTEP..3 (WSTEP = 2: with the operands read through buffer loads the
// later start gives the loads of every tile shape another k-step to land, 7B
// forward B = 1 9.49-9.53 -> 9.37-9.38 ms, seq 2048 31.4 -> 31.0 ms; WSTEP = 3
// is slower at 4096 tokens). Issuing the loads or the writes as a burst stalls the
// wave's in-order issue behind the memory queues and leaves the MFMA pipe idle
// (one wave per SIMD has nothing else to issue).
// Past the last slice the loads re-read the last slice (clamped), so every
// iteration has the same shape.
//
// Split-K: blockIdx.y selects one of gridDim.y contiguous ranges of 64-wide K
// slices (kq slices each, the last one shorter); with gridDim.y = 1 the range
// is all of K. Each split hands its partial sums to the epilogue (EpiSplit).
//
// Batches: blockIdx.z selects one of gridDim.z independent products whose
// operands start wbs and xbs halfs apart (attention backward: one per
// sequence and KV head); epilogues that care read blockIdx.z themselves.
//
// Split X rows (common.hpp): X rows hold K = 2*kw halves [hi | lo] while W
// rows hold kw; k-slice k0 reads W columns k0 mod kw, so the hi and the lo
// halves of each row meet the same weights. kw = K otherwise.
template <int FT, int TT, int WF, int WT, class Epi>
__global__ __launch_bounds__(WF* WT * 64, 1) void gemm_nt_kernel(const f16* __restrict__ W,
                                                                 const f16* __restrict__ X, int N,
                                                                 int T, int K, int kw, int kq,
                                                                 Epi epi, size_t wbs, size_t xbs) {
  W += blockIdx.z * wbs;
  X += blockIdx.z * xbs;
  constexpr int NT = WF * WT * 64;
  constexpr int WFT = FT / WF, WTT = TT / WT;
  constexpr int FM = WFT / 32, TM = WTT / 32;
  constexpr int WL = FT * 8 / NT, XL = TT * 8 / NT;
  constexpr int RSTEP = NT / 8;
  constexpr int NMF = FM * TM, NRD = FM + TM, NLD = WL + XL;
  static_assert(FM >= 1 && TM >= 1, "wave tile must be at least 32x32");
  static_assert(WL * NT == FT * 8 && XL * NT == TT * 8, "loader coverage");
  static_assert(RSTEP % 16 == 0, "loader passes must keep the LDS swizzle phase");
  static_assert(NLD <= 3 * 3 * NMF, "at most three global loads per MFMA slot");

  __shared__ f16x8 sW[2][FT * 8];
  __shared__ f16x8 sX[2][TT * 8];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int wf = wave / WT, wt = wave - wf * WT;
  const int nft = (N + FT - 1) / FT, ntt = (T + TT - 1) / TT;
  // Tile order: groups of GM weight-row panels, token tiles iterated inside a
  // group (tile = group*GM*ntt + tt*rows + row), and each XCD takes a
  // contiguous range of that order. With 8+ token tiles the 32 tiles an XCD
  // runs at a time then share 8 weight panels and 4 token panels in its L2
  // instead of 2 and 16 (7B at 4096 tokens: W1|W3 749 -> 663 us, QKV 372 ->
  // 338 us); with fewer token tiles GM = 1 (plain row-major order) measures
  // ~1% better.
  const int GM = ntt >= 8 ? 8 : 1;
  const int tile = xcd_remap(blockIdx.x, nft * ntt);
  const int grp = tile / (GM * ntt), rem = tile - grp * (GM * ntt);
  const int rows = min(GM, nft - grp * GM);
  const int tt = rem / rows, ft = grp * GM + (rem - tt * rows);
  const int f_base = ft * FT, t_base = tt * TT;

  const int r0 = tid >> 3, c0 = tid & 7;
  const int ldst = r0 * 8 + (c0 ^ lds_swz(r0));
  // Operand tiles are read through raw buffer descriptors with the sc1 (device
  // scope) policy: the loads skip L1 allocation for data this workgroup never
  // re-reads. 7B forward: B = 1 9.49-9.52 -> 9.42 ms, B = 8 56.3 -> 55.9 ms
  // against plain global loads, bit-identical. Byte offsets are 32-bit: the
  // launchers keep N*K and T*K below 2^31 elements.
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void*)W, (short)0, -1, 0x00020000);
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)X, (short)0, -1, 0x00020000);
  constexpr int kSC1 = 16;  // cache policy: sc1
  uint32_t wvo[WL], xvo[XL];  // byte offsets of this thread's 16-byte chunks at column 0
#pragma unroll
  for (int i = 0; i < WL; ++i) wvo[i] = (uint32_t)(c0 * 8 + min(f_base + r0 + RSTEP * i, N - 1) * kw) * 2u;
#pragma unroll
  for (int i = 0; i < XL; ++i) xvo[i] = (uint32_t)(c0 * 8 + min(t_base + r0 + RSTEP * i, T - 1) * K) * 2u;

  using R0 = std::integral_constant<int, 0>;
  using R1 = std::integral_constant<int, 1>;
  f16x8 wreg[2][WL], xreg[2][XL];
  auto gload = [&](auto rs, int k0) {
    constexpr int R = decltype(rs)::value;
    const int kw0 = k0 < kw ? k0 : k0 - kw;  // wave-uniform
    // per-lane row offsets in voffset, the slice's column in soffset
#pragma unroll
    for (int i = 0; i < WL; ++i)
      wreg[R][i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo[i], kw0 * 2, kSC1));
#pragma unroll
    for (int i = 0; i < XL; ++i)
      xreg[R][i] = __builtin_bit_cast(
          f16x8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xvo[i], k0 * 2, kSC1));
  };
  auto sstore = [&](auto rs) {
    constexpr int R = decltype(rs)::value;
#pragma unroll
    for (int i = 0; i < WL; ++i) sW[R][ldst + RSTEP * 8 * i] = wreg[R][i];
#pragma unroll
    for (int i = 0; i < XL; ++i) sX[R][ldst + RSTEP * 8 * i] = xreg[R][i];
  };

  f32x16 acc[FM][TM];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};

  const int khalf = lane >> 5;
  const int arow = wf * WFT + (lane & 31), brow = wt * WTT + (lane & 31);
  const int aswz = lds_swz(arow), bswz = lds_swz(brow);
  struct Frag {
    f16x8 a[FM], b[TM];
  };
  auto fread = [&](Frag& F, int buf, int ks) {
    const int c = ks * 2 + khalf;
    const int aoff = arow * 8 + (c ^ aswz), boff = brow * 8 + (c ^ bswz);
#pragma unroll
    for (int i = 0; i < FM; ++i) F.a[i] = sW[buf][aoff + i * 256];
#pragma unroll
    for (int j = 0; j < TM; ++j) F.b[j] = sX[buf][boff + j * 256];
  };
  auto mfmas = [&](const Frag& F) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < TM; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(F.a[i], F.b[j], acc[i][j], 0, 0, 0);
  };

  const int kt0 = blockIdx.y * kq;
  const int nk = min(kq, K / 64 - kt0);
  auto kslice = [&](int i) { return (kt0 + min(i, nk - 1)) * 64; };
  Frag F0, F1;
  auto iter = [&](auto rs, int kt) {
    constexpr int R = decltype(rs)::value;
    gload(rs, kslice(kt + 2));
    fread(F0, R, 0);
    fread(F1, R, 1);
    mfmas(F0);
    fread(F0, R, 2);
    mfmas(F1);
    fread(F1, R, 3);
    mfmas(F0);
    mfmas(F1);
    sstore(std::integral_constant<int, R ^ 1>{});
    // MFMA slot s = 0..4*NMF-1 in issue order
    constexpr int WSTEP = 2;
    constexpr int NSLOT = 4 * NMF, GSLOTS = 3 * NMF, WSLOTS = (4 - WSTEP) * NMF;
    __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);  // DS read, k-step 0
#pragma unroll
    for (int s = 0; s < NSLOT; ++s) {
      const int m = s % NMF;
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      if (s < 3 * NMF && m < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      if (s < GSLOTS) {
        const int g = (s + 1) * NLD / GSLOTS - s * NLD / GSLOTS;
        if (g == 1) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        if (g == 2) __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
        if (g == 3) __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);
      }
      if (s >= WSTEP * NMF) {
        const int q = s - WSTEP * NMF;
        const int w = (q + 1) * NLD / WSLOTS - q * NLD / WSLOTS;
        if (w == 1) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
        if (w == 2) __builtin_amdgcn_sched_group_barrier(0x200, 2, 0);
        if (w == 3) __builtin_amdgcn_sched_group_barrier(0x200, 3, 0);
      }
    }
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Epilogue operands read from memory: all of them before the main loop when
  // they fit in 96 registers and the tile runs one wave per SIMD anyway
  // (192x128 and larger; their latency then hides behind the K loop), else one
  // accumulator row at a time (see the epilogue).
  using AX = EpiAux<Epi>;
  using AuxT = typename AX::type;
  constexpr bool HOIST =
      !std::is_empty_v<AuxT> && FM * TM * 4 * sizeof(AuxT) <= 96 * 4 && FT * TT >= 192 * 128;
  // a staged table of up to 32 float4 per token (hd <= 128) fits in the
  // operand LDS, its first half in sW (16*FT float4) and its second in sX
  // (16*TT), when TT <= FT; staged on the 256-feature tiles, whose long
  // epilogues gain (7B QKV at 4096 tokens 424 -> 392 us, 5B at 2048 tokens
  // 105 -> 100 us), not on 128x128 (600M QKV 25.6 -> 26.6 us)
  constexpr bool STAGE = EpiStage<Epi>::value && !HOIST && TT <= FT && FT == 256;
  float4* const stab_lo = reinterpret_cast<float4*>(&sW[0][0]);
  float4* const stab_hi = reinterpret_cast<float4*>(&sX[0][0]);
  AuxT aux[HOIST ? FM : 2][TM * 4];
  auto tok = [&](int j) { return t_base + wt * WTT + j * 32 + (lane & 31); };
  auto fblk = [&](int i) { return f_base + wf * WFT + i * 32; };  // wave-uniform
  auto feat = [&](int i, int g) { return fblk(i) + 8 * g + 4 * khalf; };
  auto load_row = [&](auto ic) {
    constexpr int i = decltype(ic)::value;
    static_for<0, TM * 4>([&](auto qc) {
      constexpr int q = decltype(qc)::value;
      const int t = tok(q / 4), f = feat(i, q % 4);
      if constexpr (STAGE) {
        if (t < T && f < N)
          aux[HOIST ? i : (i & 1)][q] = epi.load_staged(stab_lo, stab_hi, t - t_base, TT, f, fblk(i));
      } else {
        if (t < T && f < N) aux[HOIST ? i : (i & 1)][q] = AX::load(epi, t, f, fblk(i));
      }
    });
  };
  if constexpr (HOIST) static_for<0, FM>([&](auto ic) { load_row(ic); });

  // nk >= 1 for every split (the launcher checks (splits - 1) * kq < K / 64)
  gload(R0{}, kslice(0));
  gload(R1{}, kslice(1));
  sstore(R0{});
  lds_barrier();
  int kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    iter(R0{}, kt);
    iter(R1{}, kt + 1);
  }
  if (kt < nk) iter(R0{}, kt);
  if constexpr (STAGE) {  // the main loop ended on a barrier: the operand LDS is free
    epi.template stage<TT, NT>(stab_lo, stab_hi, t_base, f_base, tid);
    __syncthreads();
  }

  // Epilogue over the FM x TM x 4 accumulator quads as straight-line code: a
  // loop would be left rolled once the epilogue body is large (EpiQKV on
  // 256x256 tiles), and indexing acc with a loop counter moves the whole
  // accumulator array to scratch memory. The operands that epilogues read from
  // memory (residual stream, RoPE table) were loaded before the main loop
  // (HOIST) or are loaded one accumulator row ahead of the stores: the loads
  // cannot be moved above stores that might alias them, so a load-store-load
  // chain per quad would expose the load latency once per quad.
  if constexpr (!HOIST) load_row(std::integral_constant<int, 0>{});
  // EpiRows: the token part of the output addresses once per token, the
  // (feature block, token) part once per 4 quads, both outside the quads'
  // bounds tests (they read no memory)
  constexpr bool ROWS = EpiRows<Epi>::value;
  static_assert(!ROWS || !EpiSumSq<Epi>::value, "row-addressed epilogues return nothing");
  typename EpiRows<Epi>::Tok tkj[ROWS ? TM : 1];
  if constexpr (ROWS) {
    static_for<0, TM>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      tkj[j] = epi.tok(tok(j));
    });
  }
  float lane_sq = 0.f;
  static_for<0, FM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    if constexpr (!HOIST && i + 1 < FM) load_row(std::integral_constant<int, i + 1>{});
    if constexpr (ROWS) {
      static_for<0, TM>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const auto rc = epi.row(tkj[j], fblk(i));
        static_for<0, 4>([&](auto gc) {
          constexpr int g = decltype(gc)::value, q = 4 * j + g;
          const int t = tok(j), f = feat(i, g);
          if (t < T && f < N) {
            f32x4 v;
            v.x = acc[i][j][4 * g + 0];
            v.y = acc[i][j][4 * g + 1];
            v.z = acc[i][j][4 * g + 2];
            v.w = acc[i][j][4 * g + 3];
            epi.store_row(rc, f, v, aux[HOIST ? i : (i & 1)][q], fblk(i));
          }
        });
      });
    } else {
      static_for<0, TM * 4>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        constexpr int j = q / 4, g = q % 4;
        const int t = tok(j), f = feat(i, g);
        if (t < T && f < N) {
          f32x4 v;
          v.x = acc[i][j][4 * g + 0];
          v.y = acc[i][j][4 * g + 1];
          v.z = acc[i][j][4 * g + 2];
          v.w = acc[i][j][4 * g + 3];
          if constexpr (EpiSumSq<Epi>::value)
            lane_sq += AX::apply(epi, t, f, v, aux[HOIST ? i : (i & 1)][q], fblk(i));
          else
            AX::apply(epi, t, f, v, aux[HOIST ? i : (i & 1)][q], fblk(i));
        }
      });
    }
  });
  if constexpr (EpiSumSq<Epi>::value) {
    // The main loop ended on a barrier after its last LDS reads, so the
    // operand buffers are free for the per-wave totals.
    float* red = (float*)&sW[0][0];
    const float s = wave_sum(lane_sq);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid == 0) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < WF * WT; ++w) tot += red[w];
      epi.sq_out[tile] = tot;
    }
  }
}

}  // namespace hb
