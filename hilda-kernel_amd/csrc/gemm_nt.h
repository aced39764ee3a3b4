// GEMM on gfx950 MFMA: C[M,N] = sum_k A(m,k) * B(n,k), fp32 accumulation,
// result handed to an epilogue functor in 16-byte row chunks. bf16/fp16 inputs
// run v_mfma_f32_32x32x16_{bf16,f16}; fp32 inputs (K-contiguous only) run the
// same pipeline on v_mfma_f32_32x32x2_f32, see mma_frag.
// Each operand is stored either K-contiguous (A[m][k], the "NT" layout) or
// MN-contiguous (A[k][m]); the stage tiles keep that orientation in LDS and
// the MN-contiguous ones are read with the transposing ds_read_b64_tr_b16, so
// no operand is ever transposed in memory.
//
// Layout of the work:
// * One workgroup computes a BM x BN tile with WGM x WGN waves; each wave owns a
//   (BM/WGM) x (BN/WGN) sub-tile of 32x32 v_mfma_f32_32x32x16 tiles.
// * K advances BK per stage through STAGES LDS buffers. Stage tiles are
//   [rows][BK] with the 16-byte chunk index XOR-swizzled by the row, so the
//   lanes a ds_read_b128 serves together hit distinct banks.
// * Stage tiles are filled by buffer_load_dwordx4 ... lds (no VGPR round
//   trip): each lane's 16 bytes land at LDS base + 16*lane, so the swizzle is
//   applied to the global offset each lane fetches. The buffer resource covers
//   only what the tile may read; elements past M, N or K read as zero, either
//   because they lie past the buffer's end or because the lane's offset is
//   redirected there. Nothing is clamped and nothing is read out of bounds.
// * The loads of stage kt+STAGES are issued as soon as every wave has finished
//   reading stage kt. One barrier per stage, with no memory fence (a fence
//   would drain the loads of the later stages too); vmcnt is counted by hand.
// * MFMA operands are double-buffered in registers, and the LDS reads (and the
//   global loads) are interleaved one-for-one with the MFMAs of the previous
//   sub-step by scheduling-group barriers.
// * Epilogue: the accumulators are staged through LDS (one wave row at a time)
//   and read back as 16-byte row chunks, so global stores (and the
//   read-modify-write of an fp32 accumulator) are full, coalesced 16-byte
//   accesses; all loads of a batch of chunks are issued before its stores.
//
// Workgroups are renumbered so each of the 8 XCDs walks a contiguous band of
// output tiles (grouped by GROUP_M rows of tiles), keeping the shared A/B
// panels in that XCD's L2.
//
// gemm_nt_kernel takes any layout and K; gemm_kk_kernel is the same pipeline
// specialised for two K-contiguous operands with K a multiple of the stage
// depth (64 16-bit or 32 fp32 elements), and launch() picks it whenever the
// call qualifies.
#pragma once

#include "hk_common.h"

#include <type_traits>

namespace hk {
namespace gemm {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct Shape {
  int M, N, K;
  int64_t lda, ldb;
  // optional device-side bound: with lim, M (or K when lim_k) is cut to
  // *lim - lim_off rows (K rounded up to a whole stage; the operands must hold
  // zeros there). The grid is sized for the host M; the tiles of the cut M are
  // rastered over the first workgroups (so they spread over every XCD) and the
  // rest exit.
  const int* lim = nullptr;
  int lim_off = 0;
  int lim_k = 0;
  // split-K: at most ksplit workgroups per output tile. The kernel takes
  // auto_splits() of the tiles left after the bound, so a GEMM cut short on the
  // device still fills the chip; split s sums K tiles [s * per, (s + 1) * per),
  // per = ceil(K / BK / splits), and the epilogue is told (Epi::set_split) its
  // split, the split count and the bounded M.
  int ksplit = 1;
  // K extent of each operand's stored matrix when it is shorter than K
  // (gemm_nt_kernel): k at or past it reads as zero. 0: K. A device-side K
  // bound (lim_k) also cuts both to the unrounded live count.
  int ka = 0, kb = 0;
};

// Splits for a GEMM of `tiles` output tiles and `kt` K tiles, at most max_s:
// about 512 workgroups (two a CU), every split at least 16 K tiles and non-empty.
__host__ __device__ inline int auto_splits(int tiles, int kt, int max_s) {
  if (max_s <= 1 || tiles >= 256 || tiles <= 0) return 1;
  int s = min(max_s, (512 + tiles - 1) / tiles);
  s = min(s, kt / 16);
  while (s > 1 && (kt + s - 1) / s * (s - 1) >= kt) --s;
  return s < 1 ? 1 : s;
}

// Gives a split-K epilogue its split, the split count and the bounded M; other
// epilogues have no set_split.
template <class Epi>
__device__ __forceinline__ auto apply_split(Epi& e, int s, int ns, int m, int) -> decltype(e.set_split(s, ns, m),
                                                                                          void()) {
  e.set_split(s, ns, m);
}
template <class Epi>
__device__ __forceinline__ void apply_split(Epi&, int, int, int, long) {}

// Applies Shape::lim (a uniform scalar load); kq: the K granule of the kernel.
__device__ __forceinline__ void apply_bound(Shape& g, int kq) {
  if (g.ka <= 0) g.ka = g.K;
  if (g.kb <= 0) g.kb = g.K;
  if (!g.lim) return;
  const int v = max(0, *g.lim - g.lim_off);
  if (g.lim_k) {
    g.K = min(g.K, max(kq, (v + kq - 1) / kq * kq));
    g.ka = min(g.ka, v);
    g.kb = min(g.kb, v);
  } else {
    g.M = min(g.M, v);
  }
}

// EPC: elements of the input type in a 16-byte chunk (8 for bf16/fp16, 4 for
// fp32). Stage rows of BK elements are CPR = BK / EPC chunks; a sub-step
// consumes two chunks of k per row (one per half-wave of the MFMA operand),
// one 16-bit MFMA or MPF = 4 fp32 MFMAs per fragment pair.
template <int BM_, int BN_, int BK_, int WGM_, int WGN_, int STAGES_, int GROUP_M_ = 16, int EPC_ = 8>
struct Cfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, WGM = WGM_, WGN = WGN_, STAGES = STAGES_;
  static constexpr int GROUP_M = GROUP_M_, EPC = EPC_;
  static constexpr int MPF = EPC == 8 ? 1 : 4;     // MFMA instructions per fragment pair
  static constexpr int NW = WGM * WGN, NT = NW * 64;
  static constexpr int WTM = BM / WGM, WTN = BN / WGN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int CPR = BK / EPC, RPI = 64 / CPR;  // chunks per row, rows per load instruction
  static constexpr int IA = BM / RPI / NW, IB = BN / RPI / NW;  // load instructions per wave per stage
  static constexpr int NI = IA + IB;
  static constexpr int NKS = BK / (2 * EPC);       // MFMA sub-steps per stage
  static constexpr int NR = TM + TN;               // LDS reads per sub-step
  static constexpr int STAGE = (BM + BN) * BK;     // elements per stage
  static_assert(EPC == 8 || EPC == 4, "16-bit or 32-bit elements");
  static_assert(IA * RPI * NW == BM && IB * RPI * NW == BN, "stage tile must split in 1 KiB loads");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile must be a multiple of 32x32");
  static_assert(CPR == 4 || CPR == 8, "stage rows of 64 or 128 bytes");
  static_assert(STAGES >= 2 && (STAGES - 1) * NI <= 63, "outstanding loads must fit vmcnt");
  static_assert(TM * TN >= NR, "sub-step must hold enough MFMAs to cover its reads");
  static constexpr int Q = NW >= 8 ? 2 : 4;        // MFMAs of a stage's last sub-step issued before its barrier
  static_assert(TM * TN > Q, "last sub-step split");
};

// The configuration every caller uses: 256x256 tiles, 8 waves of 128x64 (two
// per SIMD, so one wave's barrier and LDS waits overlap the other's MFMAs),
// BK=64 in two stages (128 KiB of LDS), tiles grouped 4 deep in M: the 32
// tiles an XCD runs at once then span 4 A panels and 8 B panels, which its L2
// shares better than 16 x 2 (5-12% faster). Measured fastest on the
// FusedLinearCE shapes (M, N, K in {4096, 8192, 128256}) against 4 waves of
// 128x128, BK=32 with 4 or 5 stages and groups of 6, 8, 16 and 32.
using DefaultCfg = Cfg<256, 256, 64, 2, 4, 2, 4>;

// fp32 inputs: the same tiles, waves and stage bytes (BK = 32 fp32 is the
// 128-byte stage row of BK = 64 bf16), so the LDS layout, swizzle and DMA are
// unchanged; each fragment pair feeds four fp32 MFMAs.
using F32Cfg = Cfg<256, 256, 32, 2, 4, 2, 4, 4>;

template <typename T>
using CfgFor = typename std::conditional<sizeof(T) == 4, F32Cfg, DefaultCfg>::type;

// One MFMA step of a fragment pair: a and b are 16-byte operand fragments in
// which lane l holds row l % 32 at the chunk's k offsets 8*(l/32) .. +7
// (16-bit) or 4*(l/32) .. +3 (fp32). 16-bit: one 32x32x16 MFMA. fp32: element
// q of every lane feeds 32x32x2 MFMA number q, which sums lane l's k
// (= l/32 in the instruction) over the two half-waves, so the four MFMAs
// together sum over the chunk pair's eight k (in another order than a plain
// k loop; the same products and one fp32 accumulation).
template <typename T>
__device__ __forceinline__ f32x16_t mfma32(const u32x4& a, const u32x4& b, const f32x16_t& c) {
  if constexpr (std::is_same<T, __bf16>::value) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
  } else if constexpr (std::is_same<T, _Float16>::value) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  } else {
    static_assert(std::is_same<T, float>::value, "bf16, fp16 or fp32 inputs");
    // (the whole vector is cast and then indexed: __builtin_bit_cast of a
    // single vector element, a.y, reads element 0 with this compiler)
    const f32x4_t af = __builtin_bit_cast(f32x4_t, a), bf = __builtin_bit_cast(f32x4_t, b);
    f32x16_t r = c;
    r = __builtin_amdgcn_mfma_f32_32x32x2f32(af[0], bf[0], r, 0, 0, 0);
    r = __builtin_amdgcn_mfma_f32_32x32x2f32(af[1], bf[1], r, 0, 0, 0);
    r = __builtin_amdgcn_mfma_f32_32x32x2f32(af[2], bf[2], r, 0, 0, 0);
    r = __builtin_amdgcn_mfma_f32_32x32x2f32(af[3], bf[3], r, 0, 0, 0);
    return r;
  }
}

// acc[t / TN][t % TN] += fragment pairs t of [first, first + count): one
// MFMA each for 16-bit inputs, four chained ones (the same accumulator) for
// fp32; interleaving the fp32 parts across accumulators instead needed 256
// VGPRs and spilled, the chained order 244 without spills.
template <typename T, class C>
__device__ __forceinline__ void mma_frags(f32x16_t (&acc)[C::TM][C::TN], const u32x4* fa, const u32x4* fb, int first,
                                          int count) {
#pragma unroll
  for (int t = first; t < first + count; ++t) {
    const int i = t / C::TN, j = t % C::TN;
    acc[i][j] = mfma32<T>(fb[j], fa[i], acc[i][j]);
  }
}

// two values rounded to the 16-bit type T, packed low-first into one word
template <typename T>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(lo)) |
         ((uint32_t)__builtin_bit_cast(uint16_t, from_f32<T>(hi)) << 16);
}

// XOR applied to the 16-byte chunk index of a stage row, chosen (by measuring
// ds_read_b128 rates over candidate patterns on gfx950) so that the rows read
// together at one logical chunk fall in distinct banks.
template <int CPR>
__device__ __forceinline__ int swz_xor(int row) {
  if constexpr (CPR == 8) return (row ^ (row >> 3)) & 7;
  else return (row ^ (row >> 2)) & 3;
}

// element offset of chunk kc of stage row `row`
template <class C>
__device__ __forceinline__ int swz(int row, int kc) {
  return row * C::BK + (kc ^ swz_xor<C::CPR>(row)) * C::EPC;
}

template <int GROUP_M>
__device__ __forceinline__ void tile_of_block(int pid, int nbm, int nbn, int* tm, int* tn) {
  constexpr int kXcds = 8;
  const int total = nbm * nbn;
  const int q = total / kXcds, r = total % kXcds;
  const int xcd = pid % kXcds, local = pid / kXcds;
  const int logical = xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
  const int per_group = GROUP_M * nbn;
  const int group = logical / per_group;
  const int first_m = group * GROUP_M;
  const int gsize = min(nbm - first_m, GROUP_M);
  const int in_group = logical - group * per_group;
  *tm = first_m + in_group % gsize;
  *tn = in_group / gsize;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// A buffer offset past the end of any buffer this kernel builds (the launcher
// keeps them below it) that cannot wrap when the scalar offset is added.
constexpr uint32_t kOobOffset = 0x7ff00000u;

// ---------------------------------------------------------------------------
// One operand panel: ROWS rows (of M or N) by the K range, stored K-contiguous
// (element (r, k) at p[r*ld + k]) or MN-contiguous (at p[k*ld + r]).
//
// K-contiguous stage tile: [ROWS][BK], 16-byte chunk index XOR swz_xor(row).
// A 1 KiB load instruction covers 64/CPR rows. The buffer spans the panel's
// rows (rows past the matrix read zero); chunks at or past column K are
// redirected out of the buffer.
//
// MN-contiguous stage tile: [BK][ROWS], 16-byte chunk index XOR 4*(k%4), which
// keeps the 4 k-rows x 4 chunks a 32-lane ds_read_b64_tr_b16 touches in
// distinct banks. A 1 KiB load covers 1024/(2*ROWS) k-rows. The buffer starts
// at the stage's first k-row and ends at the matrix's last element, so k-rows
// past K read zero; chunks at or past the matrix's last row are redirected.
// A fragment (32 rows x 16 k of the MFMA operand layout: lane l holds row
// l%32, k = 8*(l/32) .. +7) is two tr16 reads: within each 16-lane group the
// read returns out[j][q] = in[4q + j/4][j%4], so lane 16g+i points at k-row
// 8*(g/2) + 4h + i/4 and row 16*(g%2) + 4*(i%4).
// ---------------------------------------------------------------------------
template <typename T, class C, int ROWS, bool MN>
struct Operand {
  static constexpr int I = ROWS * C::BK * (int)sizeof(T) / 1024 / C::NW;  // 1 KiB loads per wave per stage
  static_assert(I * 1024 * C::NW == ROWS * C::BK * (int)sizeof(T), "stage tile must split in 1 KiB loads");
  static_assert(C::EPC * (int)sizeof(T) == 16, "configuration made for another element size");
  static_assert(!MN || sizeof(T) == 2, "MN-contiguous operands are 16-bit (ds_read_b64_tr_b16)");
  static_assert(!MN || ROWS / 8 >= 16, "MN-contiguous tiles need at least 16 chunks per k-row");
  static constexpr int kLoadElems = 1024 / (int)sizeof(T);  // LDS elements one 1 KiB load fills
  uint32_t voff[I];
  int key[I];  // K-contiguous: first column of the chunk in the stage; MN: first row of the chunk
  const T* p;
  int64_t ld;
  int r0, rows_valid, K;  // K: the stored matrix's K extent

  __device__ __forceinline__ void init(const T* ptr, int64_t ld_, int r0_, int nrows, int K_, int wave, int lane) {
    p = ptr;
    ld = ld_;
    r0 = r0_;
    rows_valid = min(ROWS, nrows - r0_);
    K = K_;
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const int q = (wave * I + i) * 64 + lane;  // chunk index in the stage tile
      if constexpr (!MN) {
        constexpr int CPR = C::CPR;
        const int r = q / CPR;
        key[i] = ((q % CPR) ^ swz_xor<CPR>(r)) * C::EPC;
        voff[i] = (uint32_t)(r * ld + key[i]) * sizeof(T);
      } else {
        constexpr int CPR = ROWS / 8;
        const int k = q / CPR;
        key[i] = ((q % CPR) ^ (4 * (k & 3))) << 3;
        voff[i] = (uint32_t)(k * ld + key[i]) * sizeof(T);
      }
    }
  }

  // Stage kst of this workgroup's K range, which starts at K tile kt0 (a stage
  // at or past KT, or wholly past the stored K, is a zero-length buffer: the
  // loads return zeros without touching memory) into `tile`.
  __device__ __forceinline__ void issue(T* tile, int kst, int KT, int kt0, int wave) const {
#if defined(__HIP_DEVICE_COMPILE__)
    const int k0x = (kt0 + kst) * C::BK;
    const bool live = kst < KT && k0x < K;
    const int k0 = live ? k0x : 0;
    if constexpr (!MN) {
      const int lim = K - k0;  // columns of this stage inside the matrix
      const int nrec = live ? (int)(rows_valid * ld * (int64_t)sizeof(T)) : 0;
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(p + (int64_t)r0 * ld), 0, nrec, kRsrcWord3);
#pragma unroll
      for (int i = 0; i < I; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, tile + (wave * I + i) * kLoadElems, 16,
                                                 key[i] < lim ? voff[i] : kOobOffset, k0 * (int)sizeof(T), 0, 0);
    } else {
      // from the stage's first k-row to the matrix's last element
      const int64_t span = live ? ((int64_t)(K - k0 - 1) * ld + (rows_valid > 0 ? rows_valid : 0)) * sizeof(T) : 0;
      const int nrec = (int)(span < (int64_t)kOobOffset ? span : (int64_t)kOobOffset);
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<T*>(p + (int64_t)k0 * ld + r0), 0, nrec, kRsrcWord3);
#pragma unroll
      for (int i = 0; i < I; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, tile + (wave * I + i) * kLoadElems, 16,
                                                 key[i] < rows_valid ? voff[i] : kOobOffset, 0, 0, 0);
    }
#endif
  }

  // CNT fragments for sub-step ks, rows R, R+32, ... of the tile
  template <int CNT>
  __device__ __forceinline__ void frag(const T* tile, int ks, int R, int lane, u32x4* out) const {
    if constexpr (!MN) {
      const int fr = lane & 31, fk = lane >> 5;
#pragma unroll
      for (int t = 0; t < CNT; ++t)
        out[t] = *reinterpret_cast<const u32x4*>(tile + swz<C>(R + t * 32 + fr, ks * 2 + fk));
    } else {
#if defined(__HIP_DEVICE_COMPILE__)
      typedef short v4i16 __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
      const int g = lane >> 4, i = lane & 15;
      const int kq = i >> 2;  // k % 4 of this lane's k-row
#pragma unroll
      for (int t = 0; t < CNT; ++t) {
        const int r = R + t * 32 + 16 * (g & 1) + 4 * (i & 3);
        v4i16 h[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int k = ks * 16 + 8 * (g >> 1) + 4 * hh + kq;
          const int e = k * ROWS + (((r >> 3) ^ (4 * kq)) << 3) + (r & 7);
          h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(tile + e));
        }
        const u32x2 lo = __builtin_bit_cast(u32x2, h[0]), hi = __builtin_bit_cast(u32x2, h[1]);
        out[t] = u32x4{lo.x, lo.y, hi.x, hi.y};
      }
#endif
    }
  }
};

// ---------------------------------------------------------------------------
// Epilogue contract. An epilogue functor declares
//   using Stage = float or the input type;   // how values are staged in LDS
//   using Prior = what load() returns;       // (an empty struct if kReads is false)
//   static constexpr bool kReads;            // does it read memory per chunk?
//   Prior load(row, col, n) const;           // (kReads) prior data of the chunk
//   void store(row, col, const Stage* v, n, const Prior&) const;
// and is called once per 16-byte chunk of a row: v holds 16/sizeof(Stage)
// consecutive columns starting at col, of which the first n are inside the
// matrix (n is the full chunk unless the chunk straddles column N).
//
// The accumulators go through LDS one wave row (WTM rows x BN columns) at a
// time and are read back as 16-byte row chunks, so global stores (and the
// read-modify-write of an fp32 accumulator) are full, coalesced 16-byte
// accesses; all loads of a batch of chunks are issued before its stores.
// acc[i][j] holds a transposed 32x32 tile (the MFMA is fed B then A): element
// e of a lane is row i*32 + lane%32, column j*32 + (e/4)*8 + (lane/32)*4 + e%4.
// The caller has drained every load into LDS and passed a barrier.
// ---------------------------------------------------------------------------
template <class C, class Epi>
constexpr int epilogue_lds_bytes() {
  return C::WTM * (C::BN + 16 / (int)sizeof(typename Epi::Stage)) * (int)sizeof(typename Epi::Stage);
}

template <typename T, class C, class Epi>
__device__ __forceinline__ void epilogue(const f32x16_t (&acc)[C::TM][C::TN], unsigned char* lds_raw, int m0, int n0,
                                         const Shape& g, const Epi& epi) {
  using S = typename Epi::Stage;
  constexpr int EPC = 16 / sizeof(S);  // elements per 16-byte chunk
  constexpr int LDR = C::BN + EPC;     // padded LDS row of the staged tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int fr = lane & 31, fk = lane >> 5;
  auto barrier = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  S* const st = reinterpret_cast<S*>(lds_raw);
  constexpr int CPRO = C::BN / EPC;                  // chunks per staged row
  constexpr int PER_T = C::WTM * CPRO / C::NT;       // chunks per thread per pass
  constexpr int BATCH = PER_T < 8 ? PER_T : 8;
  static_assert(C::WTM * CPRO % C::NT == 0 && PER_T % BATCH == 0, "epilogue split");
#pragma unroll 1
  for (int p = 0; p < C::WGM; ++p) {
    if (wm == p) {
#pragma unroll
      for (int i = 0; i < C::TM; ++i)
#pragma unroll
        for (int j = 0; j < C::TN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            S* dst = st + (i * 32 + fr) * LDR + wn * C::WTN + j * 32 + q * 8 + fk * 4;
            if constexpr (sizeof(S) == 4) {
              *reinterpret_cast<f32x4_t*>(dst) =
                  f32x4_t{acc[i][j][q * 4], acc[i][j][q * 4 + 1], acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]};
            } else {
              u32x2 w;
              w.x = pack2<S>(acc[i][j][q * 4], acc[i][j][q * 4 + 1]);
              w.y = pack2<S>(acc[i][j][q * 4 + 2], acc[i][j][q * 4 + 3]);
              *reinterpret_cast<u32x2*>(dst) = w;
            }
          }
    }
    barrier();
    const int rbase = m0 + p * C::WTM;
#pragma unroll
    for (int b0 = 0; b0 < PER_T; b0 += BATCH) {
      typename Epi::Prior prior[BATCH];
      if constexpr (Epi::kReads) {
#pragma unroll
        for (int u = 0; u < BATCH; ++u) {
          const int c = (b0 + u) * C::NT + tid, r = c / CPRO, col = n0 + (c % CPRO) * EPC;
          if (rbase + r < g.M && col < g.N) prior[u] = epi.load(rbase + r, col, min(EPC, g.N - col));
        }
      }
#pragma unroll
      for (int u = 0; u < BATCH; ++u) {
        const int c = (b0 + u) * C::NT + tid, r = c / CPRO, cc = c % CPRO, col = n0 + cc * EPC;
        if (rbase + r < g.M && col < g.N) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(st + r * LDR + cc * EPC);
          epi.store(rbase + r, col, reinterpret_cast<const S*>(&v), min(EPC, g.N - col), prior[u]);
        }
      }
    }
    if (p + 1 < C::WGM) barrier();
  }
}


template <typename T, class C, bool AMN, bool BMN, class Epi>
__global__ __launch_bounds__(C::NT) void gemm_nt_kernel(const T* __restrict__ A, const T* __restrict__ B, Shape g,
                                                        Epi epi) {
  constexpr int kStageBytes = C::STAGES * C::STAGE * (int)sizeof(T);
  constexpr int kEpiBytes = epilogue_lds_bytes<C, Epi>();
  constexpr int kLdsBytes = kStageBytes > kEpiBytes ? kStageBytes : kEpiBytes;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[kLdsBytes];
  T* const lds = reinterpret_cast<T*>(lds_raw);

  apply_bound(g, 8);
  const int nbm = (g.M + C::BM - 1) / C::BM, nbn = (g.N + C::BN - 1) / C::BN;
  const int tiles = nbm * nbn;
  const int KTall = (g.K + C::BK - 1) / C::BK;  // >= 1 (checked by the launcher)
  const int nsplit = auto_splits(tiles, KTall, g.ksplit);
  if ((int)blockIdx.x >= tiles * nsplit) return;  // uniform: past a device-side bound
  const int split = (int)blockIdx.x / tiles;
  int tm, tn;
  tile_of_block<C::GROUP_M>((int)blockIdx.x - split * tiles, nbm, nbn, &tm, &tn);
  const int m0 = tm * C::BM, n0 = tn * C::BN;
  int KT = KTall, kt0 = 0;
  if (nsplit > 1) {  // this split's K tiles (auto_splits keeps every split non-empty)
    const int per = (KTall + nsplit - 1) / nsplit;
    kt0 = split * per;
    KT = min(per, KTall - kt0);
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the LDS base of a load lives in M0
  const int wm = wave / C::WGN, wn = wave % C::WGN;

  // acc[i][j] holds the transposed 32x32 tile (the MFMA is fed B then A), so
  // element e of a lane is row i*32 + lane%32, column j*32 + (e/4)*8 + (lane/32)*4 + e%4:
  // four consecutive columns per group of four elements.
  f32x16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  Operand<T, C, C::BM, AMN> opa;
  Operand<T, C, C::BN, BMN> opb;
  opa.init(A, g.lda, m0, g.M, g.ka, wave, lane);
  opb.init(B, g.ldb, n0, g.N, g.kb, wave, lane);
  auto issue = [&](int stage, int kst) {
    T* la = lds + stage * C::STAGE;
    opa.issue(la, kst, KT, kt0, wave);
    opb.issue(la + C::BM * C::BK, kst, KT, kt0, wave);
  };

  u32x4 fa[2][C::TM], fb[2][C::TN];
  auto frag = [&](int stage, int ks, u32x4* a, u32x4* b) {
    const T* la = lds + stage * C::STAGE;
    opa.template frag<C::TM>(la, ks, wm * C::WTM, lane, a);
    opb.template frag<C::TN>(la + C::BM * C::BK, ks, wn * C::WTN, lane, b);
  };
  auto mma = [&](int buf, int first, int count) { mma_frags<T, C>(acc, fa[buf], fb[buf], first, count); };
  auto barrier = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // sub-steps 0 .. NKS-2 of the stage in buffer cur
  auto inner = [&](int cur) {
#pragma unroll
    for (int ks = 0; ks < C::NKS - 1; ++ks) {
      frag(cur, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      mma(ks & 1, 0, C::TM * C::TN);
#pragma unroll
      for (int t = 0; t < C::NR; ++t) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
      }
      __builtin_amdgcn_sched_group_barrier(0x008, C::MPF * C::TM * C::TN - C::NR, 0);
    }
  };
  constexpr int LB = (C::NKS - 1) & 1;  // register buffer of a stage's last sub-step
  constexpr int Q = C::Q;               // fragment pairs issued before the per-stage barrier
  constexpr int R = C::TM * C::TN - Q;  // fragment pairs after it
  constexpr int RM = R * C::MPF;        // their MFMA instructions

  // prologue: every buffer gets a stage
#pragma unroll
  for (int s = 0; s < C::STAGES; ++s) issue(s, s);
  wait_vmcnt<(C::STAGES - 1) * C::NI>();
  barrier();
  frag(0, 0, fa[0], fb[0]);

  // Straight-line body: no branch may split the MFMA chain, or the compiler
  // permutes the accumulators across the back-edge.
  for (int kt = 0; kt < KT - 1; ++kt) {
    const int cur = kt % C::STAGES;
    inner(cur);
    mma(LB, 0, Q);
    wait_vmcnt<(C::STAGES - 2) * C::NI>();  // stage kt+1 has landed
    barrier();                              // every wave is done reading stage kt
    frag((kt + 1) % C::STAGES, 0, fa[0], fb[0]);
    issue(cur, kt + C::STAGES);
    mma(LB, Q, R);
    // after the barrier: the next stage's first operand reads, then its loads,
    // each slotted behind one of the R remaining MFMAs while they last
#pragma unroll
    for (int t = 0; t < C::NR + C::NI || t < RM; ++t) {
      if (t < C::NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);             // LDS read
      else if (t < C::NR + C::NI) __builtin_amdgcn_sched_group_barrier(0x010, 1, 1);  // global->LDS load
      if (t < RM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);                  // MFMA
    }
  }
  inner((KT - 1) % C::STAGES);
  mma(LB, 0, C::TM * C::TN);
  wait_vmcnt<0>();  // the dummy loads of the tail target LDS: drain them before LDS is reused
  barrier();

  Epi e = epi;
  apply_split(e, split, nsplit, g.M, 0);
  epilogue<T, C>(acc, lds_raw, m0, n0, g, e);
}

// ---------------------------------------------------------------------------
// K % BK == 0 (every fused-linear GEMM): the same tiles and pipeline with
// nothing but MFMAs, LDS reads, DMA and scalar work in the K loop.
// * LDS holds [A stage 0][A stage 1][B stage 0][B stage 1]. A fragment's LDS
//   address is a per-lane base plus an immediate, and the K loop is unrolled
//   by two so the stage offset is an immediate too.
//   - K-contiguous operand: stage [rows][BK]; one of 16 bases (sub-step x row
//     parity; the XOR swizzle of row R + 32 i depends on i only through its
//     parity); one ds_read_b128 a fragment.
//   - MN-contiguous operand (AMN / BMN, 16-bit): stage [BK][rows], 16-byte
//     chunk index XOR 4 (k % 4); one base per fragment of the wave tile (the
//     swizzle of row R + 32 t is chunk 4 (t ^ k % 4) + ...), the sub-step and
//     half in the immediate; two ds_read_b64_tr_b16 a fragment. Its buffer is
//     rebuilt per stage at the stage's first k-row, spanning the k-rows inside
//     the stored K extent (Shape::ka / kb); chunks past the matrix's M or N are
//     redirected out of it.
// * No column masking of a K-contiguous operand: its DMA offsets are fixed per
//   lane. An odd stage count gets one trailing all-zero stage (zero-length
//   buffer loads).
// * Each sub-step issues two MFMAs, then all of the next sub-step's LDS reads,
//   then its remaining MFMAs (measured 3-4% faster than one read per MFMA).
// ---------------------------------------------------------------------------
template <typename T, class C, class Epi, bool AMN = false, bool BMN = false>
__global__ __launch_bounds__(C::NT) void gemm_kk_kernel(const T* __restrict__ A, const T* __restrict__ B, Shape g,
                                                        Epi epi) {
  static_assert(C::STAGES == 2 && C::CPR == 8, "two stages of 128-byte rows");
  static_assert(sizeof(T) == 2 || (!AMN && !BMN), "MN-contiguous operands are 16-bit (ds_read_b64_tr_b16)");
  constexpr int kStageBytes = C::STAGES * C::STAGE * (int)sizeof(T);
  constexpr int kEpiBytes = epilogue_lds_bytes<C, Epi>();
  constexpr int kLdsBytes = kStageBytes > kEpiBytes ? kStageBytes : kEpiBytes;
  static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(1024))) unsigned char lds_raw[kLdsBytes];
  T* const lds = reinterpret_cast<T*>(lds_raw);
  constexpr int kABytes = C::BM * C::BK * (int)sizeof(T);  // one A stage
  constexpr int kBBytes = C::BN * C::BK * (int)sizeof(T);
  constexpr int kBRegion = C::STAGES * kABytes;
  static_assert(kABytes + (C::TM - 1) * 32 * C::BK * (int)sizeof(T) < 65536 &&
                    kBBytes + (C::TN - 1) * 32 * C::BK * (int)sizeof(T) < 65536,
                "stage and row offsets fit the 16-bit LDS immediate");
  static_assert(kABytes + (C::BK - 4) * C::BM * (int)sizeof(T) < 65536 &&
                    kBBytes + (C::BK - 4) * C::BN * (int)sizeof(T) < 65536,
                "stage and k-row offsets fit the 16-bit LDS immediate");

  apply_bound(g, C::BK);
  const int nbm = (g.M + C::BM - 1) / C::BM, nbn = (g.N + C::BN - 1) / C::BN;
  const int tiles = nbm * nbn;
  const int nsplit = auto_splits(tiles, g.K / C::BK, g.ksplit);
  if ((int)blockIdx.x >= tiles * nsplit) return;  // uniform: past a device-side bound
  const int split = (int)blockIdx.x / tiles;
  int tm, tn;
  tile_of_block<C::GROUP_M>((int)blockIdx.x - split * tiles, nbm, nbn, &tm, &tn);
  const int m0 = tm * C::BM, n0 = tn * C::BN;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int fr = lane & 31, fk = lane >> 5;

  f32x16_t acc[C::TM][C::TN];
#pragma unroll
  for (int i = 0; i < C::TM; ++i)
#pragma unroll
    for (int j = 0; j < C::TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  int KT = g.K / C::BK, kt0 = 0;
  if (nsplit > 1) {  // this split's K tiles (auto_splits keeps every split non-empty)
    const int per = (KT + nsplit - 1) / nsplit;
    kt0 = split * per;
    KT = min(per, KT - kt0);
  }

  // K-contiguous fragment (ks, row R + 32 i) of the MFMA layout: lane l reads row R + 32 i + l%32,
  // 16-byte chunk 2 ks + l/32, stored at chunk (2 ks + l/32) ^ swz_xor(row). With R a multiple of 64,
  // swz_xor(R + 32 i + fr) = (fr & 7) ^ (fr >> 3) ^ 4 (i & 1).
  // MN-contiguous fragment t (rows R + 32 t ..): lane 16 q + i of a tr16 read points at k-row
  // 16 ks + 8 (q >> 1) + 4 h + i / 4 and row R + 32 t + 16 (q & 1) + 4 (i % 4); its chunk is row / 8
  // XOR 4 (k % 4), k % 4 = i / 4 for every (ks, h).
  constexpr int KB = AMN ? 1 : C::NKS, KBN = BMN ? 1 : C::NKS;
  uint32_t abase[KB][AMN ? C::TM : 2], bbase[KBN][BMN ? C::TN : 2];
  {
    const int sx0 = (fr & 7) ^ (fr >> 3);
    const int q = lane >> 4, ii = lane & 15, kq = ii >> 2;
    auto mn_base = [&](int R, int t, int rows) {
      const int r = R + 32 * t + 16 * (q & 1) + 4 * (ii & 3);
      const int chunk = (r >> 3) ^ (4 * kq);
      return (uint32_t)(((8 * (q >> 1) + kq) * rows + chunk * 8 + (r & 7)) * (int)sizeof(T));
    };
    if constexpr (AMN) {
#pragma unroll
      for (int t = 0; t < C::TM; ++t) {
        abase[0][t] = mn_base(wm * C::WTM, t, C::BM);
        asm volatile("" : "+v"(abase[0][t]));
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int ch = ((2 * ks + fk) ^ sx0 ^ (4 * p)) * C::EPC;
          abase[ks][p] = (uint32_t)(((wm * C::WTM + fr) * C::BK + ch) * (int)sizeof(T));
          asm volatile("" : "+v"(abase[ks][p]));  // kept in registers, not recomputed per read
        }
    }
    if constexpr (BMN) {
#pragma unroll
      for (int t = 0; t < C::TN; ++t) {
        bbase[0][t] = (uint32_t)kBRegion + mn_base(wn * C::WTN, t, C::BN);
        asm volatile("" : "+v"(bbase[0][t]));
      }
    } else {
#pragma unroll
      for (int ks = 0; ks < C::NKS; ++ks)
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const int ch = ((2 * ks + fk) ^ sx0 ^ (4 * p)) * C::EPC;
          bbase[ks][p] = (uint32_t)(kBRegion + ((wn * C::WTN + fr) * C::BK + ch) * (int)sizeof(T));
          asm volatile("" : "+v"(bbase[ks][p]));
        }
    }
  }
  // DMA: lane offsets inside the panel. K-contiguous: row r, chunk swizzled by r; the stage's
  // first column goes in the scalar offset. MN-contiguous: k-row k, chunk swizzled by k % 4, chunks
  // at or past the matrix's M (N) redirected out of the buffer; the buffer is rebuilt per stage.
  // A 1 KiB load fills kLoadElems elements of LDS.
  constexpr int IA = C::IA, IB = C::IB;
  constexpr int kLoadElems = 1024 / (int)sizeof(T);
  uint32_t va[IA], vb[IB];
  auto dma_offset = [&](bool mn, int q, int64_t ld, int rows_valid) -> uint32_t {
    if (mn) {
      constexpr int CPK = C::BM / 8;  // chunks per k-row (BM == BN)
      const int k = q / CPK, key = ((q % CPK) ^ (4 * (k & 3))) * 8;
      return key < rows_valid ? (uint32_t)(k * ld + key) * (uint32_t)sizeof(T) : kOobOffset;
    }
    const int r = q / 8;
    return (uint32_t)(r * ld + ((q % 8) ^ swz_xor<8>(r)) * C::EPC) * (uint32_t)sizeof(T);
  };
  static_assert(!(AMN || BMN) || C::BM == C::BN, "MN-contiguous stage tiles assume BM == BN");
  const int rva = min(C::BM, g.M - m0), rvb = min(C::BN, g.N - n0);
#pragma unroll
  for (int i = 0; i < IA; ++i) va[i] = dma_offset(AMN, (wave * IA + i) * 64 + lane, g.lda, rva);
#pragma unroll
  for (int i = 0; i < IB; ++i) vb[i] = dma_offset(BMN, (wave * IB + i) * 64 + lane, g.ldb, rvb);
  // K-contiguous: the panel from this split's first column, its rows inside the matrix (rows past it read
  // zero; with a split's K offset the range still ends where the panel's last row can reach).
  // MN-contiguous: the panel's columns from this split's first k-row.
  const T* const pa = AMN ? A + (int64_t)kt0 * C::BK * g.lda + m0 : A + (int64_t)m0 * g.lda + kt0 * C::BK;
  const T* const pb = BMN ? B + (int64_t)kt0 * C::BK * g.ldb + n0 : B + (int64_t)n0 * g.ldb + kt0 * C::BK;
  const int nra = AMN ? 0 : (int)(rva * g.lda * (int64_t)sizeof(T));
  const int nrb = BMN ? 0 : (int)(rvb * g.ldb * (int64_t)sizeof(T));
  if (g.ka <= 0) g.ka = g.K;
  if (g.kb <= 0) g.kb = g.K;
  const int kva = g.ka - kt0 * C::BK, kvb = g.kb - kt0 * C::BK;  // stored k-rows from this split's start

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  auto issue = [&](auto stage_c, int kst) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int st = decltype(stage_c)::value;
    const bool live = kst < KT;  // past KT: zero-length buffers, the loads return zeros
    const int k0b = live ? kst * C::BK * (int)sizeof(T) : 0;
    __amdgpu_buffer_rsrc_t ra, rb;
    int sa = k0b, sb = k0b;
    if constexpr (AMN) {
      const int kr = live ? max(0, min(C::BK, kva - kst * C::BK)) : 0;
      ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(pa + (int64_t)kst * C::BK * g.lda), 0,
                                             (int)(kr * g.lda * (int64_t)sizeof(T)), kRsrcWord3);
      sa = 0;
    } else {
      ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(pa), 0, live ? nra : 0, kRsrcWord3);
    }
    if constexpr (BMN) {
      const int kr = live ? max(0, min(C::BK, kvb - kst * C::BK)) : 0;
      rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(pb + (int64_t)kst * C::BK * g.ldb), 0,
                                             (int)(kr * g.ldb * (int64_t)sizeof(T)), kRsrcWord3);
      sb = 0;
    } else {
      rb = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(pb), 0, live ? nrb : 0, kRsrcWord3);
    }
#pragma unroll
    for (int i = 0; i < IA; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, lds + (st * kABytes) / (int)sizeof(T) + (wave * IA + i) * kLoadElems,
                                               16, va[i], sa, 0, 0);
#pragma unroll
    for (int i = 0; i < IB; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, lds + (kBRegion + st * kBBytes) / (int)sizeof(T) + (wave * IB + i) * kLoadElems, 16, vb[i], sb, 0,
          0);
#endif
  };

  u32x4 fa[2][C::TM], fb[2][C::TN];
#if defined(__HIP_DEVICE_COMPILE__)
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
  // an MN-contiguous fragment: two transposing reads (k-rows 16 ks + 4 h + ...)
  auto tr_frag = [&](uint32_t base, int off, int rows) -> u32x4 {
    v4i16 h[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
      h[hh] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (lds_v4i16*)(lds_raw + base + off + 4 * hh * rows * (int)sizeof(T)));
    const u32x2 lo = __builtin_bit_cast(u32x2, h[0]), hi = __builtin_bit_cast(u32x2, h[1]);
    return u32x4{lo.x, lo.y, hi.x, hi.y};
  };
#endif
  // fragments of sub-step ks, in the order mma() consumes them
  auto frag = [&](auto stage_c, int ks, u32x4* a, u32x4* b) {
    constexpr int st = decltype(stage_c)::value;
#pragma unroll
    for (int t = 0; t < C::TM * C::TN; ++t) {
      const int i = t / C::TN, j = t % C::TN;
      if (j == 0) {
        if constexpr (AMN) {
#if defined(__HIP_DEVICE_COMPILE__)
          a[i] = tr_frag(abase[0][i], st * kABytes + 16 * ks * C::BM * (int)sizeof(T), C::BM);
#endif
        } else {
          a[i] = *reinterpret_cast<const u32x4*>(lds_raw + abase[ks][i & 1] +
                                                 (st * kABytes + i * 32 * C::BK * (int)sizeof(T)));
        }
      }
      if (i == 0) {
        if constexpr (BMN) {
#if defined(__HIP_DEVICE_COMPILE__)
          b[j] = tr_frag(bbase[0][j], st * kBBytes + 16 * ks * C::BN * (int)sizeof(T), C::BN);
#endif
        } else {
          b[j] = *reinterpret_cast<const u32x4*>(lds_raw + bbase[ks][j & 1] +
                                                 (st * kBBytes + j * 32 * C::BK * (int)sizeof(T)));
        }
      }
    }
  };
  auto mma = [&](int buf, int first, int count) { mma_frags<T, C>(acc, fa[buf], fb[buf], first, count); };
  auto barrier = [&]() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  constexpr int NRD = (AMN ? 2 : 1) * C::TM + (BMN ? 2 : 1) * C::TN;  // LDS read instructions a sub-step
  constexpr int kPre = 2;  // MFMAs of a sub-step issued ahead of the next sub-step's reads
  static_assert(C::TM * C::TN > kPre, "sub-step split");
  // sub-steps 0 .. NKS-2 of the stage in buffer CUR
  auto inner = [&](auto stage_c) {
#pragma unroll
    for (int ks = 0; ks < C::NKS - 1; ++ks) {
      frag(stage_c, ks + 1, fa[(ks + 1) & 1], fb[(ks + 1) & 1]);
      mma(ks & 1, 0, C::TM * C::TN);
      __builtin_amdgcn_sched_group_barrier(0x008, kPre, 0);                          // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, NRD, 0);                           // LDS read
      __builtin_amdgcn_sched_group_barrier(0x008, C::MPF * C::TM * C::TN - kPre, 0);  // MFMA
    }
  };
  constexpr int LB = (C::NKS - 1) & 1;  // register buffer of a stage's last sub-step
  constexpr int Q = C::Q;               // fragment pairs issued before the per-stage barrier
  constexpr int R = C::TM * C::TN - Q;
  constexpr int RM = R * C::MPF;        // MFMA instructions after the barrier
  // stage kt in buffer CUR (stage kt+1 is landing in the other one)
  auto body = [&](auto cur_c, int kt) {
    using NX = std::integral_constant<int, decltype(cur_c)::value ^ 1>;
    inner(cur_c);
    mma(LB, 0, Q);
    wait_vmcnt<0>();  // this wave's loads of stage kt+1
    barrier();        // every wave's loads landed, every wave done reading stage kt
    frag(NX{}, 0, fa[0], fb[0]);
    issue(cur_c, kt + 2);
    mma(LB, Q, R);
#pragma unroll
    for (int t = 0; t < NRD + C::NI || t < RM; ++t) {
      if (t < NRD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);             // LDS read
      else if (t < NRD + C::NI) __builtin_amdgcn_sched_group_barrier(0x010, 1, 1);  // global->LDS load
      if (t < RM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);                  // MFMA
    }
  };

  issue(S0{}, 0);
  issue(S1{}, 1);
  wait_vmcnt<C::NI>();  // stage 0
  barrier();
  frag(S0{}, 0, fa[0], fb[0]);
  const int KT2 = KT + (KT & 1);
  // Straight-line body: no branch may split the MFMA chain, or the compiler
  // permutes the accumulators across the back-edge.
  for (int kt = 0; kt + 2 < KT2; kt += 2) {
    body(S0{}, kt);
    body(S1{}, kt + 1);
  }
  body(S0{}, KT2 - 2);
  inner(S1{});
  mma(LB, 0, C::TM * C::TN);
  wait_vmcnt<0>();  // the trailing zero-length loads target LDS: drain them before it is reused
  barrier();
  Epi e = epi;
  apply_split(e, split, nsplit, g.M, 0);
  epilogue<T, C>(acc, lds_raw, m0, n0, g, e);
}

// Returns 0, or -1 with the error set for shapes the kernel does not take.
// AMN / BMN: the operand is stored MN-contiguous (A[k][m], B[k][n]) instead of
// K-contiguous (A[m][k], B[n][k]); lda / ldb are the leading dimensions of
// whichever layout is used.
//
// ka / kb (0: K): the K extent of A's / B's stored matrix when shorter than K
// (its k past that read as zero; general kernel only). ksplit: see Shape.
template <typename T, class C = CfgFor<T>, bool AMN = false, bool BMN = false, class Epi>
int launch(const T* A, const T* B, int M, int N, int K, int64_t lda, int64_t ldb, Epi epi, hipStream_t st,
           const int* lim = nullptr, int lim_off = 0, bool lim_k = false, int ksplit = 1, int ka = 0, int kb = 0) {
  static_assert(sizeof(T) == 2 || (!AMN && !BMN), "fp32 operands must be K-contiguous");
  if (M == 0 || N == 0) return 0;
  if (K <= 0) {
    set_error("gemm: K (%d) must be positive", K);
    return -1;
  }
  if (ka < 0 || kb < 0 || ka > K || kb > K) {
    set_error("gemm: operand K extents (%d, %d) outside [0, K = %d]", ka, kb, K);
    return -1;
  }
  if (ksplit > 1 && lim_k) {
    set_error("gemm: split-K with a device-side K bound is not supported");
    return -1;
  }
  auto check = [&](bool mn, int rows, int64_t ld, const char* name) {
    if (mn) {
      if (rows % 8 != 0 || ld % 8 != 0 || ld < rows) {
        set_error("gemm: MN-contiguous %s needs rows (%d) and ld (%lld) multiples of 8, ld >= rows", name, rows,
                  (long long)ld);
        return false;
      }
      if ((int64_t)C::BK * ld * (int64_t)sizeof(T) >= (int64_t)kOobOffset) {
        set_error("gemm: a %d-row stage of %s exceeds the 2 GiB buffer range", C::BK, name);
        return false;
      }
    } else {
      if (K % 8 != 0 || ld % 8 != 0 || ld < K) {
        set_error("gemm: K-contiguous %s needs K (%d) and ld (%lld) multiples of 8, ld >= K", name, K, (long long)ld);
        return false;
      }
      if ((int64_t)C::BM * ld * (int64_t)sizeof(T) >= (int64_t)kOobOffset) {
        set_error("gemm: a %d-row panel of %s exceeds the 2 GiB buffer range", C::BM, name);
        return false;
      }
    }
    return true;
  };
  if (!check(AMN, M, lda, "A") || !check(BMN, N, ldb, "B")) return -1;
  Shape g{M, N, K, lda, ldb, lim, lim_off, lim_k ? 1 : 0, ksplit < 1 ? 1 : ksplit, ka, kb};
  const int64_t blocks = (int64_t)((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN) * g.ksplit;
  if constexpr (C::STAGES == 2 && C::CPR == 8 && C::BM == C::BN) {
    // The pipelined kernel: K a whole number of stages; a K-contiguous operand read to K (its extent must be
    // K), an MN-contiguous one to its extent (k-rows past it read zero).
    const bool a_ok = AMN || ka == 0 || ka == K;
    const bool b_ok = BMN || kb == 0 || kb == K;
    if (K % C::BK == 0 && a_ok && b_ok) {
      hipLaunchKernelGGL((gemm_kk_kernel<T, C, Epi, AMN, BMN>), dim3((unsigned)blocks), dim3(C::NT), 0, st, A, B, g,
                         epi);
      return check_launch("gemm_kk_kernel");
    }
  }
  hipLaunchKernelGGL((gemm_nt_kernel<T, C, AMN, BMN, Epi>), dim3((unsigned)blocks), dim3(C::NT), 0, st, A, B, g,
                     epi);
  return check_launch("gemm_nt_kernel");
}

}  // namespace gemm
}  // namespace hk
