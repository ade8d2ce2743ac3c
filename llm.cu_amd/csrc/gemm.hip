// gemm.hip — skinny "NT" GEMM on fp16 MFMA (v_mfma_f32_16x16x32_f16) for
// gfx950, plus the layout kernels (fragment packing, transposes,
// conversions, the bit-exact int8 quantizer) and the split-K reduction used
// by the standalone GEMM entry points.
//
// Every frozen-weight product of the training step is expressed as
// C = A * B^T with both operands contiguous along the reduction dimension:
// the forward uses W [out, in] as B, the backward (dX = dY * W) uses the
// pre-transposed copy W^T [in, out] the library keeps next to W.  This is the
// MI355X-native replacement for the reference's three fp32 32x32-tiled
// kernels (src/kernels/matmul.cu:8-138): matmul_forward (NT), matmul_nn
// (dX) and, for LoRA, matmul_tn.
//
// Work decomposition.  The step's activations have few rows (T = 128 at the
// headline shape), so every weight element is used T times: the kernel is
// HBM-bound on the weight stream.  B operands are stored fragment-packed
// (packed_index in common.h): each wave streams its NF*16 weight rows as
// contiguous 1 KB loads straight into MFMA operand registers through a
// register ring (RING - 1 k-steps of 32 ahead).  The A tile of all MF*16 rows
// is staged through LDS in 64-wide K chunks (double-buffered, in MFMA
// fragment order so every ds_read_b128 is a contiguous conflict-free 1 KB)
// and shared by the NW waves; the next chunk's A loads are issued a chunk of
// MFMA work before they are stored.  K is split across workgroups (split-K)
// so a launch fills the CUs; the fp32 split partials are summed in split
// order by the consuming row epilogue (deterministic), and the standalone
// GEMM entry points reduce them with reduce_lora.  Measured on MI355X
// (per-workgroup timestamps): the in-loop weight stream runs at 2.6-3.8 TB/s,
// and each launch pays ~5 us of fixed latency (launch, the first A/B round
// trip, the partial stores), which four-wave 128-column tiles at about 3/4 of
// a workgroup per CU balance best against the partial traffic; deeper B
// rings and A prefetch distances measured no faster.
#include <math.h>
#include <stdlib.h>
#include <type_traits>

#include "ops.h"

namespace llmt {

static int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  return v && *v ? atoi(v) : dflt;
}

namespace {

#define LLMT_INLINE __attribute__((always_inline))

constexpr int KSTEP = 32;  // k per MFMA

template <int V>
using IC = std::integral_constant<int, V>;

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }
constexpr int lcm_c(int a, int b) { return a / gcd_c(a, b) * b; }

// Packed int8 weights are stored biased, byte = x + 128 (x ^ 0x80; written by
// pack_i8), so that fp16 bits 0x64 | byte read as 1024 + x + 128, exact.
// v_perm_b32 picks bytes 0-3 from its second source and 4-7 from its
// first: each output dword [b_i, 0x64, b_i+1, 0x64] is one instruction.
__device__ __forceinline__ half8 i8x8_to_h8(u32x2 raw) {
  constexpr unsigned k64 = 0x64646464u, s01 = 0x04010400u, s23 = 0x04030402u;
  u32x4 bits;
  bits[0] = __builtin_amdgcn_perm(k64, raw[0], s01);
  bits[1] = __builtin_amdgcn_perm(k64, raw[0], s23);
  bits[2] = __builtin_amdgcn_perm(k64, raw[1], s01);
  bits[3] = __builtin_amdgcn_perm(k64, raw[1], s23);
  const half8 h = __builtin_bit_cast(half8, bits);
  return h - (_Float16)1152.0f;
}

// One workgroup: output tile (MF*16) x (NW*NF*16) over k-steps [s0, s1) of
// its split.  The A tile goes through LDS in chunks of CHS k-steps (two LDS
// buffers); chunk c + ADIST is loaded into registers while chunk c is
// multiplied, so an A load has ADIST chunks of MFMA work to land.  B
// fragments stream through a RING-slot register ring, RING - 1 k-steps
// ahead.  The main loop body covers UC chunks so that every LDS buffer,
// A register set and ring slot index is a compile-time constant.  Chunks
// and k-steps past the end are clamped loads multiplied by zeroed B
// fragments (branch-free: the compiler then keeps the newer loads in flight
// across every wait).  With I8 a segment may be int8 (dequantised in
// registers at MFMA time, optionally times a per-k scale loaded alongside).
template <int MF, int NF, int NW, int CHS, int RING, int ADIST, bool I8>
__global__ __launch_bounds__(NW * 64) void gemm_nt_kernel(const GemmArgs g) {
  constexpr int MT = MF * 16;
  constexpr int NT = NW * 64;
  constexpr int CH = CHS * KSTEP;
  constexpr int PIECES = MT * (CH / 8);  // 16-byte A pieces per chunk
  constexpr int APT = (PIECES + NT - 1) / NT;
  constexpr int UC = lcm_c(lcm_c(2, ADIST), lcm_c(RING, CHS) / CHS);
  static_assert(ADIST == 1 || ADIST == 2, "A prefetch distance is one or two chunks");
  // A chunk in LDS in MFMA fragment order: fragment (k-step q, m-tile mi) is
  // 1 KB at (q * MF + mi) * 512 halves with lane l's 8 halves at l * 8, so
  // every ds_read_b128 of a wave is one contiguous, conflict-free 1 KB, and
  // the staging writes (thread i -> piece i) are contiguous too.
  __shared__ __attribute__((aligned(16))) _Float16 As[2][MT * CH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int m0 = blockIdx.z * MT;
  const int ksteps = g.K / KSTEP;
  const int s0 = (int)((long long)blockIdx.y * ksteps / g.split);
  const int s1 = (int)((long long)(blockIdx.y + 1) * ksteps / g.split);
  const int nst = s1 - s0;
  const int nch = (nst + CHS - 1) / CHS;

  const char* bptr[NF];
  int bi8[NF];
  int ncol[NF];
  const _Float16* cscale[NF];
  const _Float16* kscale[NF];
  bool valid[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    const int nn = (blockIdx.x * NW + wave) * NF * 16 + f * 16;
    ncol[f] = nn;
    valid[f] = nn < g.N;
    int s = 0;
#pragma unroll
    for (int i = 1; i < 4; ++i)
      if (i < g.nseg && nn >= g.seg_start[i]) s = i;
    const BSeg& sg = g.seg[s];
    // Invalid fragments read row block 0 of their segment (in bounds) and
    // are never stored.
    const long long rb16 = valid[f] ? (nn - g.seg_start[s]) >> 4 : 0;
    const int i8 = I8 ? sg.is_i8 : 0;
    bptr[f] = (const char*)sg.ptr + ((rb16 * ksteps) * 512 + lane * 8) * (i8 ? 1 : 2);
    bi8[f] = i8;
    cscale[f] = sg.colscale ? sg.colscale + (nn - g.seg_start[s]) : nullptr;
    kscale[f] = (I8 && sg.kscale) ? sg.kscale + (lane >> 4) * 8 : nullptr;
  }

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int f = 0; f < NF; ++f) acc[i][f] = floatx4{0.f, 0.f, 0.f, 0.f};

  u32x4 ra[ADIST][APT];
  u32x4 rb[RING][NF];
  u32x4 rk[RING][NF];

  auto load_a = [&](int c, auto R) LLMT_INLINE {
    constexpr int set = decltype(R)::value;
    const int kb = (s0 + min(c, nch - 1) * CHS) * KSTEP;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + i * NT;  // LDS piece: fragment idx / 64, lane idx % 64
      if (PIECES % NT == 0 || idx < PIECES) {
        const int fr = idx >> 6, l = idx & 63;
        const int q = fr / MF, mi = fr % MF;
        const int r = mi * 16 + (l & 15);
        const int k = min(kb + q * KSTEP + (l >> 4) * 8, g.K - 8);
        ra[set][i] = *reinterpret_cast<const u32x4*>(g.A + (long long)(m0 + r) * g.lda + k);
      }
    }
  };
  auto store_a = [&](auto R, auto BUF) LLMT_INLINE {
    constexpr int set = decltype(R)::value;
    constexpr int buf = decltype(BUF)::value;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int idx = tid + i * NT;
      if (PIECES % NT == 0 || idx < PIECES)
        *reinterpret_cast<u32x4*>(&As[buf][idx * 8]) = ra[set][i];
    }
  };
  auto load_b = [&](int j, auto S) LLMT_INLINE {
    constexpr int st = decltype(S)::value;
    const long long ss = s0 + min(j, nst - 1);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (I8 && bi8[f]) {
        const u32x2 q = *reinterpret_cast<const u32x2*>(bptr[f] + ss * 512);
        rb[st][f] = u32x4{q[0], q[1], 0u, 0u};
        if (kscale[f]) rk[st][f] = *reinterpret_cast<const u32x4*>(kscale[f] + ss * KSTEP);
      } else {
        rb[st][f] = *reinterpret_cast<const u32x4*>(bptr[f] + ss * 1024);
      }
    }
  };
  auto bfrag = [&](int f, auto S) LLMT_INLINE -> half8 {
    constexpr int st = decltype(S)::value;
    half8 h;
    if (I8 && bi8[f]) {
      h = i8x8_to_h8(u32x2{rb[st][f][0], rb[st][f][1]});
      if (kscale[f]) {
        h = h * __builtin_bit_cast(half8, rk[st][f]);
      }
    } else {
      h = __builtin_bit_cast(half8, rb[st][f]);
    }
    return h;
  };
  // k-step j = (chunk base cb + u) * CHS + q: ring slot (u * CHS + q) % RING
  // and LDS buffer u % 2 are static within the unrolled body.
  auto kstep = [&](int cb, auto U, auto Q) LLMT_INLINE {
    constexpr int u = decltype(U)::value;
    constexpr int q = decltype(Q)::value;
    constexpr int pos = u * CHS + q;
    const int j = (cb + u) * CHS + q;
    load_b(j + RING - 1, IC<(pos + RING - 1) % RING>{});
    const bool live = j < nst;
    half8 b[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      b[f] = bfrag(f, IC<pos % RING>{});
      if (!live) b[f] = half8{};
    }
#pragma unroll
    for (int mi = 0; mi < MF; ++mi) {
      const half8 a =
          *reinterpret_cast<const half8*>(&As[u % 2][((q * MF + mi) * 64 + lane) * 8]);
#pragma unroll
      for (int f = 0; f < NF; ++f) acc[mi][f] = mfma16(a, b[f], acc[mi][f]);
    }
  };
  auto chunk = [&](int cb, auto U) LLMT_INLINE {
    constexpr int u = decltype(U)::value;
    // chunk cb + u + ADIST goes to register set (u + ADIST) % ADIST = u % ADIST
    load_a(cb + u + ADIST, IC<u % ADIST>{});
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... Q>(std::integer_sequence<int, Q...>) LLMT_INLINE {
      (kstep(cb, IC<u>{}, IC<Q>{}), ...);
    }(std::make_integer_sequence<int, CHS>{});
    // chunk cb + u + 1 was loaded ADIST - 1 chunks ago into set (u + 1) % ADIST
    store_a(IC<(u + 1) % ADIST>{}, IC<(u + 1) % 2>{});
    __syncthreads();
  };

  if (nst > 0) {
    load_a(0, IC<0>{});
    if constexpr (ADIST == 2) load_a(1, IC<1>{});
    [&]<int... P>(std::integer_sequence<int, P...>) LLMT_INLINE {
      (load_b(P, IC<P>{}), ...);
    }(std::make_integer_sequence<int, RING - 1>{});
    store_a(IC<0>{}, IC<0>{});
    __syncthreads();
    // The unrolled body stops at the last chunk (uniform exit), so a deep
    // ring costs no padded MFMA work on short K ranges.
    for (int c = 0; c < nch; c += UC) {
      [&]<int... U>(std::integer_sequence<int, U...>) LLMT_INLINE {
        ((c + U < nch ? (chunk(c, IC<U>{}), true) : false) && ...);
      }(std::make_integer_sequence<int, UC>{});
    }
  }

  float* C = g.C + (long long)blockIdx.y * g.split_stride;
  float cs[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f) cs[f] = cscale[f] ? (float)cscale[f][lane & 15] : 1.0f;
#pragma unroll
  for (int f = 0; f < NF; ++f) {
    if (!valid[f]) continue;
    const int col = ncol[f] + (lane & 15);
#pragma unroll
    for (int mi = 0; mi < MF; ++mi) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + mi * 16 + (lane >> 4) * 4 + v;
        C[(long long)row * g.ldc + col] = acc[mi][f][v] * cs[f];
      }
    }
  }
  if (g.rowstats) {
    // each row's (max, sum exp) over the workgroup's NW NF 16 columns: a
    // wave's pair from its 16-lane groups, the NW waves merged in wave order
    float2* sh = reinterpret_cast<float2*>(&As[0][0]);  // [MT][NW]
    static_assert(MT * NW * 8 <= 2 * MT * CH * 2, "pairs fit in the A buffers");
    __syncthreads();  // every wave is past its last A fragment read
#pragma unroll
    for (int mi = 0; mi < MF; ++mi)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float x[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) x[f] = valid[f] ? acc[mi][f][v] * cs[f] : -INFINITY;
        const float2 p = softmax_pair16<NF>(x);
        if ((lane & 15) == 0) sh[(mi * 16 + (lane >> 4) * 4 + v) * NW + wave] = p;
      }
    __syncthreads();
    for (int r = tid; r < MT; r += NT) {
      float m = -INFINITY, s = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) softmax_merge(m, s, sh[r * NW + w].x, sh[r * NW + w].y);
      g.rowstats[(long long)(m0 + r) * gridDim.x + blockIdx.x] = make_float2(m, s);
    }
  }
}

constexpr int BM = 256, BCH = 2;  // large-tile rows; k-steps per big_tiles() K quantum

// LDS-DMA kernel for the large-M GEMMs: the operands go from global memory
// straight into LDS (global_load_lds: lane l's 16 bytes land at offset 16 l
// of the wave's block; a fragment-packed fp16 fragment is 1 KB in lane order
// and an int8 one 512 B, moved by the first 32 lanes, so both arrive in MFMA
// fragment order with no register staging and no LDS store phase), through
// an S-stage ring of 32-wide K chunks: chunks up to c + S - 1 are in flight
// while chunk c is multiplied.  Each workgroup of eight waves owns a 256 x 256
// tile (2 x 4 waves of 128 x 64, 32 accumulator fragments a wave; the
// four-wave form with 128 x 128 a wave measured 12-20% slower at the C4
// shapes).  The fragments run one chunk ahead in registers: while the MFMAs
// of chunk c issue, chunk c + 1's fragments are read from LDS (each A
// fragment register refilled right after its last MFMA), so LDS latency and
// the int8 dequantisation (exact int8 -> fp16 from the biased bytes, one
// v_perm_b32 and one v_pk_add_f16 a dword, times the per-k scale if any)
// leave the critical path (C4 dX
// GEMMs 187.5 -> 183.5 us, the tail-folded ones 2-3% faster).  The waits are
// explicit: vmcnt counts this thread's DMA issues, which complete in order,
// and a plain s_barrier (no fence, which would drain every load) publishes
// the chunk to the other waves.
__device__ __forceinline__ void dma16(const void* src, _Float16* lds_blk) {
  __builtin_amdgcn_global_load_lds(src, (void __attribute__((address_space(3)))*)lds_blk, 16, 0, 0);
}
// s_waitcnt with vmcnt = N (lgkmcnt and expcnt left free), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}


// TL: a trailing fp16 segment `tail` of at most 64 rows (the LoRA A or B^T
// rows of a projection, output columns tail_c0 ..) rides along: its 16-row
// fragment f is computed by the workgroups of column tile f, over their row
// block and K range (two extra MFMAs a wave per chunk, the fragment's 1 KB
// a chunk moved by eight lanes of every wave), instead of a separate launch
// that streamed the whole activation matrix again.
template <bool I8, bool KS, int S, int WNN, bool GLU = false, bool TL = false>
__global__ __launch_bounds__(WNN * 128) void gemm_dma_kernel(const GemmArgs g, int g_order,
                                                             const BSeg tail, int tail_c0) {
  // WNN waves across N (2: four waves of 128 x 128; 4: eight waves of 128 x 64)
  constexpr int NW = 2 * WNN, WC = 256 / WNN, NFR = WC / 16;  // wave columns, fragments
  constexpr int FPW = 16 / NW;                                 // A (and B) fragments each wave moves
  constexpr int ABYTES = 256 * KSTEP * 2;
  constexpr int BBYTES = 256 * KSTEP * (I8 ? 1 : 2);
  constexpr int KSBYTES = KS ? 256 : 0;
  constexpr int TOFF = ABYTES + BBYTES + KSBYTES;              // tail fragment slot
  constexpr int SBYTES = TOFF + (TL ? 1024 : 0);
  constexpr int OPS = 2 * FPW + (KS ? 1 : 0) + (TL ? 1 : 0);   // DMA issues per chunk per thread
  static_assert(!(TL && GLU), "no tail with the SwiGLU epilogue");
  static_assert(!TL || WNN == 4, "the tail fragment is split over four column waves");
  __shared__ __attribute__((aligned(1024))) char smem[S * SBYTES];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WNN, wn = wave % WNN;
  const int ntn = (g.N + 255) / 256, ntm = g.M / 256;
  int t = blockIdx.x, sidx = blockIdx.y, nsp = g.split, tn0 = 0, ntn_r = ntn;
  if (g.split_col > 0) {
    // column tiles [0, ntc) unsplit (workgroups 0 .. ntc ntm - 1), then the
    // rest split in two over K (split 0 of every such tile, then split 1)
    const int ntc = g.split_col / 256, nfull = ntc * ntm;
    if (t < nfull) {
      nsp = 1;
      sidx = 0;
      ntn_r = ntc;
    } else {
      t -= nfull;
      nsp = 2;
      tn0 = ntc;
      ntn_r = ntn - ntc;
      sidx = t / (ntn_r * ntm);
      t -= sidx * (ntn_r * ntm);
    }
  }
  const int nwg = ntn_r * ntm;
  if (g_order >= 1 && nwg % 8 == 0) t = (t % 8) * (nwg / 8) + t / 8;
  // Consecutive t of one XCD walk GM row blocks per column step, so the 32
  // tiles an XCD runs at once share 4 A row blocks and 8 B column blocks in
  // its L2 (not 1 and 32): the logits GEMM 3.05 -> 2.88 ms at C4.
  const int GM = ntm % 4 == 0 ? 4 : ntm % 2 == 0 ? 2 : 1;
  const int grp = t / (GM * ntn_r), tr = t % (GM * ntn_r);
  const int tm = grp * GM + tr % GM, tn = tn0 + tr / GM;
  const int n0 = tn * 256, m0 = tm * 256;
  const int ksteps = g.K / KSTEP;
  const int c0 = (int)((long long)sidx * ksteps / nsp);
  const int c1 = (int)((long long)(sidx + 1) * ksteps / nsp);

  // issue pointers: wave w moves A fragments FPW w .. and B fragments FPW w ..
  // of every chunk (plus, with KS, k-scales through lane 0 of waves 0-3)
  const _Float16* asrc =
      g.A + (long long)(m0 + wave * FPW * 16 + (lane & 15)) * g.lda + (lane >> 4) * 8;
  const long long astep = 16LL * g.lda;
  const BSeg& sg = g.seg[0];
  constexpr int ES = I8 ? 1 : 2;
  const char* bsrc = (const char*)sg.ptr + (long long)lane * 16;  // lanes < 32 for int8
  // SwiGLU pairs: tile fragment f is gate (f even) or up (f odd) row block
  // 8 tn + f / 2, so a wave's fragments 2 p and 2 p + 1 cover the same columns
  long long boff[FPW];
#pragma unroll
  for (int j = 0; j < FPW; ++j) {
    const int f = wave * FPW + j;
    const int rb = GLU ? (f & 1) * (g.glu >> 4) + tn * 8 + (f >> 1)
                       : min((n0 >> 4) + f, (g.N >> 4) - 1);
    boff[j] = (long long)rb * ksteps * 512 * ES;
  }
  const _Float16* ksrc = KS ? sg.kscale + (wave & 3) * 8 : nullptr;
  // tail fragment of this column tile (tiles past the last fragment load the
  // last one, unused, so every wave issues the same number of DMAs)
  const int ntf = TL ? tail.rows / 16 : 0;
  const bool has_tail = TL && tn < ntf;
  const _Float16* tsrc =
      TL ? (const _Float16*)tail.ptr + (long long)min(tn, ntf - 1) * ksteps * 512 + (wave * 8 + lane) * 8
         : nullptr;
  auto issue = [&](int c) LLMT_INLINE {
    const int cc = min(c, c1 - 1);
    char* st = smem + (c % S) * SBYTES;
#pragma unroll
    for (int j = 0; j < FPW; ++j)
      dma16(asrc + j * astep + cc * KSTEP, reinterpret_cast<_Float16*>(st + (wave * FPW + j) * 1024));
#pragma unroll
    for (int j = 0; j < FPW; ++j) {
      const char* src = bsrc + boff[j] + (long long)cc * 512 * ES;
      _Float16* dst = reinterpret_cast<_Float16*>(st + ABYTES + (wave * FPW + j) * 512 * ES);
      if constexpr (I8) {
        if (lane < 32) dma16(src, dst);
      } else {
        dma16(src, dst);
      }
    }
    if constexpr (KS) {
      if (lane == 0 && wave < 4)
        dma16(ksrc + (long long)cc * KSTEP, reinterpret_cast<_Float16*>(st + ABYTES + BBYTES + wave * 16));
      else if (lane == 0)  // keep the per-thread DMA count uniform (a harmless re-read)
        dma16(ksrc + (long long)cc * KSTEP, reinterpret_cast<_Float16*>(st + ABYTES + BBYTES + 64 + (wave & 3) * 16));
    }
    if constexpr (TL) {  // wave w moves bytes 128 w .. 128 w + 127 of the fragment
      if (lane < 8) dma16(tsrc + (long long)cc * 512, reinterpret_cast<_Float16*>(st + TOFF + wave * 128));
    }
  };

  floatx4 acc[8][NFR];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < NFR; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  // tail: this wave's rows 16 (2 wn + j) .. of its 128-row half
  floatx4 acc_t[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};

  // Fragments one chunk ahead: after the barrier that publishes chunk
  // c + 1, each A fragment register of chunk c is refilled from chunk c + 1
  // right after its last MFMA, and chunk c + 1's B bytes (and k-scales,
  // tail fragment) are read at the top, dequantised after the last MFMA;
  // so LDS latency sits under the MFMAs and the registers stay one set.
  half8 a[8], b[NFR], bt, btn, ksn, at[2], atn[2];
  u32x2 bn8[NFR];
  half8 bn16[NFR];
  auto read_b = [&](const char* st) LLMT_INLINE {
    if constexpr (KS) ksn = *reinterpret_cast<const half8*>(st + ABYTES + BBYTES + (lane >> 4) * 16);
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      const int fr = wn * NFR + j;
      if constexpr (I8)
        bn8[j] = *reinterpret_cast<const u32x2*>(st + ABYTES + fr * 512 + lane * 8);
      else
        bn16[j] = *reinterpret_cast<const half8*>(st + ABYTES + fr * 1024 + lane * 16);
    }
    if constexpr (TL) {
      // the tail's fragment and the two A fragments it meets (rows
      // 16 (2 wn + j) of the wave's half), read on their own so the tail
      // MFMAs need no register selection
      btn = *reinterpret_cast<const half8*>(st + TOFF + lane * 16);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        atn[j] = *reinterpret_cast<const half8*>(st + (wm * 8 + 2 * wn + j) * 1024 + lane * 16);
    }
  };
  auto take_b = [&]() LLMT_INLINE {
#pragma unroll
    for (int j = 0; j < NFR; ++j) {
      if constexpr (I8) {
        b[j] = i8x8_to_h8(bn8[j]);
        if constexpr (KS) b[j] = b[j] * ksn;
      } else {
        b[j] = bn16[j];
      }
    }
    if constexpr (TL) {
      bt = btn;
      at[0] = atn[0];
      at[1] = atn[1];
    }
  };
  auto read_a = [&](const char* st, int i) LLMT_INLINE {
    a[i] = *reinterpret_cast<const half8*>(st + (wm * 8 + i) * 1024 + lane * 16);
  };
#pragma unroll
  for (int c = 0; c < S; ++c) issue(c0 + c);
  static_assert((S - 1) * OPS < 64, "vmcnt range");
  wait_vm<(S - 1) * OPS>();
  __builtin_amdgcn_s_barrier();
  {
    const char* st = smem + (c0 % S) * SBYTES;
    read_b(st);
#pragma unroll
    for (int i = 0; i < 8; ++i) read_a(st, i);
    take_b();
  }
  for (int c = c0; c < c1; ++c) {
    // vmcnt: chunk c + 1 landed; lgkmcnt 0: this wave's reads of chunk c
    // returned, so after the barrier chunk c's slot takes chunk c + S
    constexpr int N = (S - 2) * OPS;
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
    __builtin_amdgcn_s_barrier();
    issue(c + S);
    const char* st = smem + ((c + 1) % S) * SBYTES;
    read_b(st);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int j = 0; j < NFR; ++j) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
      read_a(st, i);
    }
    // the order the loop states: chunk c + 1's B (and scale, tail) reads
    // first, then per row its MFMAs followed by the read that refills its A
    // register (left alone, the compiler sank all eight A reads below the
    // last MFMA, exposing their latency at the barrier)
    __builtin_amdgcn_sched_group_barrier(0x100, (I8 ? NFR / 2 : NFR) + (KS ? 1 : 0) + (TL ? 3 : 0), 0);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, NFR, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    if constexpr (TL) {
      if (has_tail) {
        acc_t[0] = mfma16(at[0], bt, acc_t[0]);
        acc_t[1] = mfma16(at[1], bt, acc_t[1]);
      }
    }
    // the dequantisation stays below the rows: hoisted up to the B reads
    // (as the compiler otherwise does with part of it) it waits on them
    // right at the top of the chunk.  VALU may not cross; MFMA, LDS, SALU
    // and memory instructions may.
    __builtin_amdgcn_sched_barrier(0);
    take_b();
  }
  wait_vm<0>();

  float* C = g.C + (long long)sidx * g.split_stride;
  const _Float16* cs = sg.colscale;
  if constexpr (GLU) {
    float sgu[NFR];
#pragma unroll
    for (int jj = 0; jj < NFR / 2; ++jj) {
      const int col = (tn * 8 + ((wn * NFR) >> 1) + jj) * 16 + (lane & 15);
      sgu[2 * jj] = cs ? (float)cs[col] : 1.0f;
      sgu[2 * jj + 1] = cs ? (float)cs[g.glu + col] : 1.0f;
    }
    const int col0 = (tn * 8 + ((wn * NFR) >> 1)) * 16 + (lane & 15);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const long long row = m0 + wm * 128 + i * 16 + (lane >> 4) * 4 + v;
        _Float16* grow = g.gu16 + row * (2LL * g.glu) + col0;
        _Float16* arow = g.glu16 + row * g.ldglu + col0;
#pragma unroll
        for (int jj = 0; jj < NFR / 2; ++jj) {
          const float gt = acc[i][2 * jj][v] * sgu[2 * jj], up = acc[i][2 * jj + 1][v] * sgu[2 * jj + 1];
          grow[16 * jj] = (_Float16)gt;
          grow[g.glu + 16 * jj] = (_Float16)up;
          arow[16 * jj] = (_Float16)(gt * sigmoid_rcp(gt) * up);
        }
      }
    return;
  }
  if constexpr (TL) {
    if (has_tail) {
      const int col = tail_c0 + tn * 16 + (lane & 15);
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + wm * 128 + (2 * wn + j) * 16 + (lane >> 4) * 4 + v;
          C[(long long)row * g.ldc + col] = acc_t[j][v];
        }
    }
  }
  float scj[NFR];
#pragma unroll
  for (int j = 0; j < NFR; ++j) {
    const int col = n0 + wn * WC + j * 16 + (lane & 15);
    scj[j] = cs && col < g.N ? (float)cs[col] : 1.0f;
  }
  // store addresses: a wave-uniform row base plus one 32-bit lane offset
  // for all stores (the compiler then steps one 64-bit address by ldc, one
  // add a store instead of a 64-bit multiply-add and an add: the fp16
  // logits GEMM at C4 2429 -> 2370 us; the same for the SwiGLU epilogue's
  // fp16 stores measured 1% slower)
  const int lo = (lane >> 4) * 4 * g.ldc + (lane & 15);
  float* const Cw = C + (long long)(m0 + wm * 128) * g.ldc + n0 + wn * WC;
#pragma unroll
  for (int j = 0; j < NFR; ++j) {
    if (n0 + wn * WC + j * 16 >= g.N) continue;  // N % 16 == 0: whole fragments
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float* const Cr = Cw + (long long)(i * 16 + v) * g.ldc + j * 16;
        Cr[lo] = acc[i][j][v] * scj[j];
      }
  }
  if (g.rowstats) {
    // each row's (max, sum exp) over the tile's 256 columns: a wave's pair
    // over its WC columns from its 16-lane groups, the WNN waves of a row
    // block merged in order (the ring is free: every DMA has landed)
    float2* sh = reinterpret_cast<float2*>(smem);  // [256 rows][WNN]
    __syncthreads();  // every wave is past its last fragment read
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float x[NFR];
#pragma unroll
        for (int j = 0; j < NFR; ++j) {
          const int col = n0 + wn * WC + j * 16 + (lane & 15);
          x[j] = col < g.N ? acc[i][j][v] * scj[j] : -INFINITY;
        }
        const float2 p = softmax_pair16<NFR>(x);
        if ((lane & 15) == 0) sh[(wm * 128 + i * 16 + (lane >> 4) * 4 + v) * WNN + wn] = p;
      }
    __syncthreads();
    for (int r = tid; r < 256; r += WNN * 128) {
      float m = -INFINITY, s = 0.f;
#pragma unroll
      for (int w = 0; w < WNN; ++w) softmax_merge(m, s, sh[r * WNN + w].x, sh[r * WNN + w].y);
      g.rowstats[(long long)(m0 + r) * ntn + tn] = make_float2(m, s);
    }
  }
}

// Skinny fp16 kernel fed by DMA (the T = 128 training step): a 128 x BN
// output tile (BN = 16 NB) per workgroup of eight waves, K split over
// blockIdx.x (the fastest grid index) in 64-wide stages.  Wave w = 4 kg + wr computes rows
// 32 wr .. 32 wr + 31 x all BN columns over k half kg (32 of the 64) of
// every stage, so each SIMD runs two waves whose LDS reads and MFMAs
// interleave; the two halves' sums meet in LDS at the end (kg 1 hands its
// accumulators to kg 0, which stores).  Both operands move global -> LDS with
// buffer loads that have an LDS destination, 16 bytes a lane: A as 128-byte
// row pieces (8 lanes a row, so each stage touches every A cache line once;
// the 16-byte pieces are XOR-swizzled by row so the fragment reads are
// bank-conflict free; wave w moves rows 16 w .. 16 w + 15), B as the 1 KB
// fragment of k half kg of each fragment-packed row block (row blocks wr,
// wr + 4, ..; one wave-uniform descriptor per row block, the stage offset a
// scalar).  An S-stage ring (A 16 KB + B 2 NB KB a stage) keeps S - 1 stages
// in flight; stage c is waited for with an explicit vmcnt (the loads of later
// stages stay in flight) and a plain barrier, the last S - 1 stages wait for
// all.  A wave reads all fragments of its stage half before its MFMAs.
// Measured on MI355X (C2 shapes, back to back): 5-15% below the four-wave
// form with the same tiles; the partial tiles and the first round trip set
// the rest of the cost at this M.  Columns past N load row block 0 of the
// first segment (in bounds) and are not stored.
constexpr int kRsrcWord3 = 0x00020000;  // raw buffer, 32-bit data format
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void buffer_lds16(__amdgpu_buffer_rsrc_t rs, void* lds, unsigned voff,
                                             unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kRsrcWord3);
}
// slot of 16-byte piece p (0..7) of A row r in a stage
__device__ __forceinline__ int a_slot(int r, int p) { return p ^ ((r >> 1) & 7); }

// GLU: fragment f of the tile is the gate (f even) or up (f odd) row block of
// the same 16 columns (split 1, one segment, N = 2 glu); the epilogue writes
// [gate | up] and fp16(silu(gate) * up) as the large-tile kernel's.
template <int S, int NB, bool GLU = false>
__global__ __launch_bounds__(512) void gemm_skinny_kernel(const GemmArgs g) {
  constexpr int AB = 16384;                  // A bytes per stage
  constexpr int SB = AB + NB * 2048;         // bytes per stage
  constexpr int BPW = (NB + 3) / 4;          // B row blocks a wave moves at most (wr, wr + 4, ..)
  static_assert(4 * 2 * NB * 64 * 16 <= S * SB, "k-half exchange fits in the ring");
  __shared__ __attribute__((aligned(1024))) char smem[S * SB];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = wave & 3, kg = wave >> 2;
  // grid = (split, column tile, row tile): the split is the fastest index,
  // so workgroup b (on XCD b % 8) of split s reads A's K slice s, and that
  // slice reaches only the XCDs running split s (one of eight at split 8 or
  // 16) instead of every XCD's L2 -- the lm_head dX at C2 had fetched its
  // 39 MB A operand eight times over
  const int ct = blockIdx.y, sp = blockIdx.x;
  const int n0 = ct * (NB * 16), m0 = blockIdx.z * 128;
  const int ksteps = g.K / KSTEP;
  const int nst = g.K / 64;
  const int c0 = (int)((long long)sp * nst / g.split);
  const int c1 = (int)((long long)(sp + 1) * nst / g.split);

  // A: wave w moves rows 16 w .. 16 w + 15 (two 1 KB pieces of 8 rows)
  const __amdgpu_buffer_rsrc_t ars =
      make_rsrc(g.A + (long long)m0 * g.lda, (unsigned)(128u * g.lda * 2u));
  unsigned aoff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = 8 * (2 * wave + i) + (lane >> 3);
    aoff[i] = (unsigned)((r * g.lda + a_slot(r, lane & 7) * 8) * 2);
  }
  const int nbw = (NB - wr + 3) / 4;  // row blocks this wave moves
  __amdgpu_buffer_rsrc_t brs[BPW];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    if constexpr (GLU) {
      const int f = min(wr + 4 * i, NB - 1);
      const long long rb = (f & 1) * (g.glu >> 4) + (long long)ct * (NB / 2) + (f >> 1);
      brs[i] = make_rsrc((const _Float16*)g.seg[0].ptr + rb * ksteps * 512, (unsigned)(ksteps * 1024u));
      continue;
    }
    const int nn = n0 + 16 * min(wr + 4 * i, NB - 1);
    int s = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q < g.nseg && nn >= g.seg_start[q]) s = q;
    const long long rb16 = nn < g.N ? (nn - g.seg_start[s]) >> 4 : 0;
    brs[i] = make_rsrc((const _Float16*)g.seg[s].ptr + rb16 * ksteps * 512, (unsigned)(ksteps * 1024u));
  }
  auto issue = [&](int c) LLMT_INLINE {
    char* st = smem + (c % S) * SB;
#pragma unroll
    for (int i = 0; i < 2; ++i) buffer_lds16(ars, st + (2 * wave + i) * 1024, aoff[i], c * 128u);
#pragma unroll
    for (int i = 0; i < BPW; ++i)
      if (i < nbw)
        buffer_lds16(brs[i], st + AB + ((wr + 4 * i) * 2 + kg) * 1024, lane * 16u + kg * 1024u,
                     c * 2048u);
  };
  // stage c complete: only the later stages' loads (2 + nbw a stage) may be pending
  auto wait_stage = [&]() LLMT_INLINE {
    switch (nbw) {
      case 0: wait_vm<(S - 2) * 2>(); break;
      case 1: wait_vm<(S - 2) * 3>(); break;
      default: wait_vm<(S - 2) * 4>(); break;
    }
  };
  // A fragment reads: row 16 (2 wr + i) + c of the stage, k half kg, halves 8 g..
  const int arow0 = 16 * (2 * wr) + (lane & 15);
  int aread[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = arow0 + 16 * i;
    aread[i] = r * 128 + a_slot(r, 4 * kg + (lane >> 4)) * 16;
  }

  floatx4 acc[2][NB];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int c = c0; c < c1 && c < c0 + S - 1; ++c) issue(c);
  for (int c = c0; c < c1; ++c) {
    if (c + S - 1 < c1) {
      wait_stage();
      __builtin_amdgcn_s_barrier();
      issue(c + S - 1);
    } else {
      wait_vm<0>();
      __builtin_amdgcn_s_barrier();
    }
    asm volatile("" ::: "memory");
    const char* st = smem + (c % S) * SB;
    half8 a[2], b[NB];
#pragma unroll
    for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const half8*>(st + aread[i]);
#pragma unroll
    for (int j = 0; j < NB; ++j)
      b[j] = *reinterpret_cast<const half8*>(st + AB + (j * 2 + kg) * 1024 + lane * 16);
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int i = 0; i < 2; ++i) acc[i][j] = mfma16(a[i], b[j], acc[i][j]);
    asm volatile("" ::: "memory");
  }

  // k half 1 hands its sums to k half 0 (the ring is free: every load has
  // landed and every wave is past its last fragment read)
  wait_vm<0>();
  __syncthreads();
  floatx4* xch = reinterpret_cast<floatx4*>(smem) + wr * (2 * NB * 64);
  if (kg == 1) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < NB; ++j) xch[(i * NB + j) * 64 + lane] = acc[i][j];
  }
  __syncthreads();
  if (kg == 1) return;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[i][j] += xch[(i * NB + j) * 64 + lane];

  float* C = g.C + (long long)sp * g.split_stride;
  if constexpr (GLU) {
    const _Float16* cs = g.seg[0].colscale;
#pragma unroll
    for (int jj = 0; jj < NB / 2; ++jj) {
      const int col = (ct * (NB / 2) + jj) * 16 + (lane & 15);
      const float sg = cs ? (float)cs[col] : 1.0f, su = cs ? (float)cs[g.glu + col] : 1.0f;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const long long row = m0 + (2 * wr + i) * 16 + (lane >> 4) * 4 + v;
          const float gt = acc[i][2 * jj][v] * sg, up = acc[i][2 * jj + 1][v] * su;
          g.gu16[row * (2LL * g.glu) + col] = (_Float16)gt;
          g.gu16[row * (2LL * g.glu) + g.glu + col] = (_Float16)up;
          g.glu16[row * g.ldglu + col] = (_Float16)(gt * sigmoid_rcp(gt) * up);
        }
    }
    return;
  }
  // a wave-uniform row base plus one 32-bit lane offset for every store
  const int lo = (lane >> 4) * 4 * g.ldc + (lane & 15);
  float* const Cw = C + (long long)(m0 + 2 * wr * 16) * g.ldc + n0;
#pragma unroll
  for (int j = 0; j < NB; ++j) {
    const int nn = n0 + 16 * j;
    if (nn >= g.N) continue;
    int s = 0;
#pragma unroll
    for (int q = 1; q < 4; ++q)
      if (q < g.nseg && nn >= g.seg_start[q]) s = q;
    const _Float16* cs = g.seg[s].colscale;
    const int col = nn + (lane & 15);
    const float sc = cs ? (float)cs[col - g.seg_start[s]] : 1.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float* const Cr = Cw + (long long)(i * 16 + v) * g.ldc + 16 * j;
        Cr[lo] = acc[i][j][v] * sc;
      }
  }
}

template <int MF, int NF, int NW, int CHS, int RING, int ADIST>
hipError_t launch_cfg(const GemmArgs& g, hipStream_t st) {
  const int ncols = NW * NF * 16;
  dim3 grid((g.N + ncols - 1) / ncols, g.split, g.M / (MF * 16));
  bool i8 = false;
  for (int i = 0; i < g.nseg; ++i) i8 = i8 || g.seg[i].is_i8;
  if (i8)
    hipLaunchKernelGGL((gemm_nt_kernel<MF, NF, NW, CHS, RING, ADIST, true>), grid, dim3(NW * 64), 0,
                       st, g);
  else
    hipLaunchKernelGGL((gemm_nt_kernel<MF, NF, NW, CHS, RING, ADIST, false>), grid, dim3(NW * 64),
                       0, st, g);
  return hipGetLastError();
}

// The register-staged kernel's pipeline: 4 waves a workgroup, 2 k-steps an
// LDS chunk, a 4-slot B ring, A prefetched one chunk ahead (measured the
// fastest of the variants tried on the logits GEMM and the int8 GEMMs).
constexpr int kNF = 2, kNW = 4;

template <int MF>
hipError_t launch_mf(const GemmArgs& g, hipStream_t st) {
  return launch_cfg<MF, kNF, kNW, 2, 4, 1>(g, st);
}

// Fixed-order split-K reduction fused with the LoRA up-projections:
//   out[m][n] = sum_s part[s][m][n] + lscale * sum_r h[m][r] * M_p(r, n - c0_p)
// for n inside adapter p's column range (adapters may share columns: each
// one covering n adds its term), where h (the rank-16 LoRA activations,
// x A^T forward or dy B backward) is itself a set of extra columns of the same
// GEMM, reduced here first, per 16-row block, into LDS.  M_p is B [n, 16]
// (forward: y += s h B^T) or A [16, n] (backward: dx += s dh A).
// Workgroup: 16 rows x 64 columns; thread = one row x four columns.  The
// kernel is latency-bound (the partials were just written), so every load
// it needs (adapter block, h partials, column partials; RB splits at a time)
// is issued before the first sum; sums run in split order (deterministic).
constexpr int RB = 16;  // partial loads in flight per thread

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// sum_s p[s * ss] for s < split, in order, RB loads in flight
__device__ __forceinline__ float4 sum_splits(const float* p, int split, long long ss) {
  float4 v = *reinterpret_cast<const float4*>(p);
  for (int k = 1; k < split; k += RB) {
    float4 x[RB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
      x[i] = *reinterpret_cast<const float4*>(p + (long long)min(k + i, split - 1) * ss);
#pragma unroll
    for (int i = 0; i < RB; ++i)
      if (k + i < split) v = add4(v, x[i]);
  }
  return v;
}

__global__ __launch_bounds__(256) void reduce_lora_kernel(const ReduceArgs a) {
  __shared__ float hs[16][3 * 16 + 4];
  __shared__ float ms[3][16][64 + 1];  // this block's 64 columns of each adapter matrix
  const int m0 = blockIdx.y * 16;
  const int cb = blockIdx.x * 64;
  const int tid = threadIdx.x;
  // Adapter column ranges are multiples of 64 wide and aligned: a block is
  // entirely inside or outside each of them.
  int inside = 0;
  for (int q = 0; q < a.nlora; ++q)
    if (cb >= a.up[q].c0 && cb < a.up[q].c0 + a.up[q].n) inside |= 1 << q;
  // adapter blocks -> registers (12 values per thread per adapter)
  float mreg[3][4];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    if (!(inside >> q & 1)) continue;
    const LoraUp& u = a.up[q];
    const int jb = cb - u.c0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = tid + 256 * e;  // 0..1023
      mreg[q][e] = u.is_B ? u.M[(long long)(jb + (i >> 4)) * 16 + (i & 15)]
                          : u.M[(long long)(i >> 6) * u.n + jb + (i & 63)];
    }
  }
  // h partials: thread -> (row tid / 12, 4 h columns), 192 threads
  const int nh4 = 4 * a.nlora;  // float4 groups of h per row
  float4 hv = make_float4(0.f, 0.f, 0.f, 0.f);
  const bool hthread = inside && tid < 16 * nh4;
  const int hr = hthread ? tid / nh4 : 0, hg = hthread ? tid % nh4 : 0;
  if (hthread)
    hv = sum_splits(a.part + (long long)(m0 + hr) * a.ldp + a.up[hg >> 2].hcol + (hg & 3) * 4,
                    a.split, a.ss);
  const int t = tid >> 4;
  const int cc = (tid & 15) * 4;
  const int c = cb + cc;
  const bool live = c < a.N;
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (live) v = sum_splits(a.part + (long long)(m0 + t) * a.ldp + c, a.split, a.ss);
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    if (!(inside >> q & 1)) continue;
    const bool isB = a.up[q].is_B;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = tid + 256 * e;
      if (isB) ms[q][i & 15][i >> 4] = mreg[q][e];
      else ms[q][i >> 6][i & 63] = mreg[q][e];
    }
  }
  if (hthread) {
    float* h = &hs[hr][(hg >> 2) * 16 + (hg & 3) * 4];
    h[0] = hv.x; h[1] = hv.y; h[2] = hv.z; h[3] = hv.w;
  }
  __syncthreads();
  if (!live) return;
  for (int q = 0; q < a.nlora; ++q) {
    if (!(inside >> q & 1)) continue;
    float l0 = 0.f, l1 = 0.f, l2 = 0.f, l3 = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float h = hs[t][q * 16 + r];
      l0 += h * ms[q][r][cc];
      l1 += h * ms[q][r][cc + 1];
      l2 += h * ms[q][r][cc + 2];
      l3 += h * ms[q][r][cc + 3];
    }
    v.x += a.lscale * l0;
    v.y += a.lscale * l1;
    v.z += a.lscale * l2;
    v.w += a.lscale * l3;
  }
  if (a.out_scale != 0.f && a.out_scale != 1.f) {
    v.x *= a.out_scale;
    v.y *= a.out_scale;
    v.z *= a.out_scale;
    v.w *= a.out_scale;
  }
  *reinterpret_cast<float4*>(a.out + (long long)(m0 + t) * a.ldo + c) = v;
}

// Pack rows [row0, row0 + R) x k [k0, k0 + C) of a fragment-packed B operand
// (row length K) from a row-major source (leading dimension lds): if
// transpose, element (i, j) of the destination block is src[j][i], else
// src[i][j].  One thread per 8-element piece; C % 8 == 0, k0 % 8 == 0.
// int8: zs (may be NULL) is the fp16 scale of each source row; a row whose
// scale is 0 is stored as zeros, so the packed values agree with the
// dequantised weights whichever side applies the scale.
template <typename T>
__global__ void pack_kernel(const T* __restrict__ src, long long lds, int transpose, int R, int C,
                            T* __restrict__ dst, long long K, int row0, int k0,
                            const _Float16* __restrict__ zs) {
  const long long np = (long long)R * (C / 8);
  for (long long p = (long long)blockIdx.x * blockDim.x + threadIdx.x; p < np;
       p += (long long)gridDim.x * blockDim.x) {
    int i, jp;
    if (transpose) {  // consecutive threads: consecutive destination rows
      i = (int)(p % R);
      jp = (int)(p / R);
    } else {
      i = (int)(p / (C / 8));
      jp = (int)(p % (C / 8));
    }
    T v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int sr = transpose ? jp * 8 + e : i;  // source row
      v[e] = transpose ? src[(long long)sr * lds + i] : src[(long long)i * lds + jp * 8 + e];
      if (zs && zs[sr] == (_Float16)0.0f) v[e] = T(0);
    }
    T* d = dst + packed_index(row0 + i, k0 + jp * 8, K);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (std::is_same_v<T, int8_t>)
        d[e] = (int8_t)((uint8_t)v[e] ^ 0x80u);  // biased: byte = x + 128
      else
        d[e] = v[e];
    }
  }
}

// 64x64 tiles through LDS; 256 threads.
__global__ void transpose_f16_kernel(const _Float16* __restrict__ src, int rows, int cols, int lds,
                                     _Float16* __restrict__ dst, int ldd) {
  __shared__ _Float16 tile[64][65];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = src[(long long)gr * lds + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < rows) dst[(long long)gc * ldd + gr] = tile[tx][c];
  }
}

__global__ void transpose_i8_kernel(const int8_t* __restrict__ src, int rows, int cols, int lds,
                                    int8_t* __restrict__ dst, int ldd) {
  __shared__ int8_t tile[64][68];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int gr = r0 + r, gc = c0 + tx;
    if (gr < rows && gc < cols) tile[r][tx] = src[(long long)gr * lds + gc];
  }
  __syncthreads();
  for (int c = ty; c < 64; c += 4) {
    const int gc = c0 + c, gr = r0 + tx;
    if (gc < cols && gr < rows) dst[(long long)gc * ldd + gr] = tile[tx][c];
  }
}

__global__ void f32_to_f16_kernel(const float* __restrict__ s, _Float16* __restrict__ d, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    d[i] = (_Float16)s[i];
}

__global__ void copy_rows_f16_kernel(const _Float16* __restrict__ s, int rows, int cols, int lds,
                                     _Float16* __restrict__ d, int ldd) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)rows * cols) return;
  const int r = (int)(i / cols), c = (int)(i % cols);
  d[(long long)r * ldd + c] = s[(long long)r * lds + c];
}

__global__ void fill_f32_kernel(float* d, float v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    d[i] = v;
}

// src/kernels/quantize.cu:8-44, bit-exact: scale = max|w|/127 (IEEE fp32
// division), inv = 1/scale, q = rint(clamp(w*inv, -127, 127)) with
// round-half-to-even (v_rndne_f32).  One workgroup of 256 per row.
__global__ void quantize_rows_kernel(const float* __restrict__ w, int cols, int8_t* __restrict__ q,
                                     float* __restrict__ scale) {
  __shared__ float red[4];
  const long long base = (long long)blockIdx.x * cols;
  float m = 0.f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) m = fmaxf(m, fabsf(w[base + c]));
  m = block_max<4>(m, red);
  const float sc = m / 127.0f;
  if (threadIdx.x == 0) scale[blockIdx.x] = sc;
  const float inv = sc > 0.f ? 1.0f / sc : 0.f;
  for (int c = threadIdx.x; c < cols; c += blockDim.x) {
    float v = w[base + c] * inv;
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[base + c] = (int8_t)rintf(v);
  }
}

__global__ void f32_scale_to_f16_kernel(const float* s, _Float16* d, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) d[i] = (_Float16)s[i];
}

inline int grid1d(size_t n, int bs, int cap = 65536) {
  size_t g = (n + bs - 1) / bs;
  return (int)(g > (size_t)cap ? cap : (g == 0 ? 1 : g));
}

}  // namespace

void gemm_finalize_segments(GemmArgs& g) {
  int s = 0;
  for (int i = 0; i < g.nseg; ++i) {
    g.seg_start[i] = s;
    s += g.seg[i].rows;
  }
  for (int i = g.nseg; i <= 4; ++i) g.seg_start[i] = s;
  g.N = s;
}

// Split-K factor: enough (column tiles x splits) workgroups for about one
// per CU, without splits shorter than 4 k-steps of 32.  Fewer splits means
// fewer fp32 partials to reduce.
// DMA skinny kernel (fp16 weights, M % 128 == 0; LLMT_GEMM_SKINNY_STAGES = 0
// selects the register-staged kernel).  Plan: 64-column tiles (48 when that
// fills more of the GPU) and the most splits that keep the grid within one
// wave of the 256 CUs (a second, partial wave costs more than the extra
// partials); at least two 64-wide stages a split.  Wider tiles at the same
// grid size write proportionally more fp32 partials and measured slower.  Very wide outputs with no split (the lm_head logits) keep the
// register-staged kernel, measured faster there.  LLMT_GEMM_SKINNY_NB forces
// the width for tuning.
static int skinny_stages() { return env_int("LLMT_GEMM_SKINNY_STAGES", 4); }
struct SkinnyPlan {
  int nb, split;
};
static SkinnyPlan skinny_plan(int M, int N, int K) {
  const int frags = (N + 15) / 16, mt = M / 128;
  const int forced = env_int("LLMT_GEMM_SKINNY_NB", 0);
  // Workgroups aimed for: one per CU, except that short reductions
  // (K <= 4096) aim for 192, i.e. fewer K splits.  Each split is an fp32
  // [M, N] partial that the row pass after the GEMM reads back, and at these
  // K those partials come close to the weight bytes (7 splits of K = 2048:
  // 0.9x); measured on the whole M = 128 training step, 5.23 -> 5.19 ms, with
  // the GEMMs alone 0-8% slower.
  const int target = K <= 4096 ? 192 : 256;
  SkinnyPlan best{0, 0};
  int best_w = 0;
  // Very long reductions (the logits' dX, K = V): every column tile re-reads
  // its K range of A, so 128-column tiles halve that traffic (163 -> 141 us
  // at M = 128, N = 2048, K = 151936); elsewhere 64/48-column tiles.
  const bool wide = K >= 32768;
  for (int nb : {4, 3, 2, 6, 8}) {
    if (!forced && (wide ? nb != 8 : (nb != 4 && nb != 3))) continue;
    if (forced && nb != forced) continue;
    const int tiles = (frags + nb - 1) / nb * mt;
    int split = target / tiles;
    if (split > K / 128) split = K / 128;
    if (split < 1) split = 1;
    const int w = tiles * split;
    if (w <= target && w > best_w) {
      best = {nb, split};
      best_w = w;
    }
  }
  if (!best.nb) best = {forced ? forced : 4, 1};
  return best;
}
static bool skinny_ok(int M, int N, int K) {
  return M % 128 == 0 && K % 64 == 0 && skinny_stages() != 0 && (N + 15) / 16 < 2048;
}

// The 256 x 256 tile kernel takes GEMMs with many rows; the skinny kernels
// everything else.
static bool big_tiles(int M, int K) { return M >= 1024 && M % BM == 0 && K % (BCH * KSTEP) == 0; }
static bool use_big_tiles(const GemmArgs& g) {
  return big_tiles(g.M, g.K) && g.N >= 16 && g.split <= (g.K / (BCH * KSTEP));
}
// Large-tile split-K: the one of 1, 2, 4 with the least modelled time.  A
// wave of tiles costs (0.54 + K / split / 1024) units, one unit being a
// 256 x 256 tile's 1024-deep K slice; each split past the first adds an fp32
// [M, N] partial that the GEMM writes and its consumer reads back, M N / 3.15e7
// units.  (Fitted on MI355X at M = 4096: int8 tiles of K = 1024 and 2048 took
// 49 and 81 us, and the SwiGLU backward read 100 MB of extra partial in
// 25 us; so N = 6144, K = 2048 runs unsplit in 1.5 waves, 384 tiles, while the
// 128-tile GEMMs split in two.)
// A trailing LoRA segment of <= 64 columns rides in the main launch (its
// fragments on the first column tiles' workgroups), so it adds no tiles.
static int big_split(int M, int N, int K, int max_split) {
  const int nmain = (N % 256 != 0 && N % 64 != 0) ? N - N % 64 : N;
  const int tiles = (nmain + 255) / 256 * (M / BM);
  const double partial = (double)M * N / 3.15e7;
  int best = 1;
  double best_t = 1e300;
  for (int split = 1; split <= 4 && split <= max_split && split <= K / (BCH * KSTEP) / 4;
       split *= 2) {
    const double t = ceil(tiles * split / 256.0) * (0.54 + K / (1024.0 * split)) +
                     (split - 1) * partial;
    if (t < best_t) best_t = t, best = split;
  }
  return best;
}

// The DMA large-tile kernel carries the SwiGLU epilogue: 256-wide tiles over
// 8 waves, gate/up fragment pairs per wave.
int gemm_rowstats_tiles(const GemmArgs& g) {
  if (g.split != 1 || g.nseg != 1 || g.glu || g.N < 16) return 0;
  if (use_big_tiles(g)) return (g.N + 255) / 256;  // gemm_dma_kernel tiles
  return (g.N + kNW * kNF * 16 - 1) / (kNW * kNF * 16);  // gemm_nt_kernel workgroups
}

bool gemm_glu_ok(int M, int I, int K, bool i8) {
  if (big_tiles(M, K))
    return I % 128 == 0 && big_split(M, 2 * I, K, 64) == 1;
  // the skinny kernel, 32 gate + 32 up columns a workgroup, split 1
  return !i8 && skinny_ok(M, 2 * I, K) && I % 32 == 0;
}

// The last wave of an unsplit large-tile GEMM: with tiles = full waves of
// the 256 CUs plus r more (r <= 128, whole column tiles), the last r tiles
// run as 2 r half-K workgroups, so the launch takes 1 + 1/2 wave-times of a
// tile instead of 2 (C4's down-projection dX: 384 tiles).  Their partial
// is an extra fp32 [M, r/ntm x 256] the consumer reads back.
int gemm_split_col(int M, int N, int K) {
  if (!big_tiles(M, K) || N % 256 || big_split(M, N, K, 64) != 1 ||
      K / (BCH * KSTEP) < 8)
    return 0;
  const int ntm = M / BM, ntn = N / 256, tiles = ntm * ntn;
  const int rest = tiles % 256;
  if (tiles < 256 || rest == 0 || rest > 128 || rest % ntm) return 0;
  return (ntn - rest / ntm) * 256;
}

int gemm_pick_split(int M, int N, int K, int max_split) {
  if (big_tiles(M, K)) return big_split(M, N, K, max_split);
  if (skinny_ok(M, N, K)) {
    const int split = skinny_plan(M, N, K).split;
    return split > max_split ? max_split : split;
  }
  // Partials grow with the workgroup count: about 3/4 of the CUs for the
  // layer GEMMs, two waves of CUs for the very long lm_head dX reduction.
  const int target = K > 16384 ? 512 : 192;
  constexpr int min_steps = 4;
  const int mt = (M % 128 == 0) ? M / 128 : 1;
  constexpr int tn = kNW * kNF * 16;
  const int ntiles = (N + tn - 1) / tn * mt;
  int split = (target + ntiles / 2) / ntiles;
  const int kmax = (K / KSTEP) / min_steps;
  if (split > kmax) split = kmax;
  if (split > max_split) split = max_split;
  if (split < 1) split = 1;
  return split;
}

// M % 128 == 0 with fp16 weights: the DMA-fed skinny kernel, 128 x BN tiles.
// LDS of an S-stage ring of NB-fragment tiles within the 160 KB of a CU
template <int S, int NB>
constexpr bool skinny_fits = S * (16384 + NB * 2048) <= 160 * 1024;

template <int S>
static void launch_skinny(const GemmArgs& g, int nb, hipStream_t st) {
  const dim3 grid(g.split, (g.N + nb * 16 - 1) / (nb * 16), g.M / 128);
  switch (nb) {
    case 2: hipLaunchKernelGGL((gemm_skinny_kernel<S, 2>), grid, dim3(512), 0, st, g); break;
    case 3: hipLaunchKernelGGL((gemm_skinny_kernel<S, 3>), grid, dim3(512), 0, st, g); break;
    case 6:
      if constexpr (skinny_fits<S, 6>)
        hipLaunchKernelGGL((gemm_skinny_kernel<S, 6>), grid, dim3(512), 0, st, g);
      break;
    case 8:
      if constexpr (skinny_fits<S, 8>)
        hipLaunchKernelGGL((gemm_skinny_kernel<S, 8>), grid, dim3(512), 0, st, g);
      break;
    default: hipLaunchKernelGGL((gemm_skinny_kernel<S, 4>), grid, dim3(512), 0, st, g); break;
  }
}
static hipError_t launch_m128(const GemmArgs& g, hipStream_t st) {
  bool i8 = false;
  for (int i = 0; i < g.nseg; ++i) i8 = i8 || g.seg[i].is_i8;
  if (i8 || g.rowstats || !skinny_ok(g.M, g.N, g.K) || g.split > g.K / 64)
    return launch_mf<8>(g, st);
  const int nb = skinny_plan(g.M, g.N, g.K).nb;
  const int stages = skinny_stages();
  if (stages == 6 && nb > 4) {
    set_error("gemm_nt: %d-stage skinny ring of %d fragments exceeds the LDS", stages, nb);
    return hipErrorInvalidValue;
  }
  switch (stages) {
    case 3: launch_skinny<3>(g, nb, st); break;
    case 5: launch_skinny<5>(g, nb, st); break;
    case 6: launch_skinny<6>(g, nb, st); break;
    default: launch_skinny<4>(g, nb, st); break;
  }
  return hipGetLastError();
}

const char* gemm_kernel_name(const GemmArgs& g) {
  if (use_big_tiles(g)) {
    const int last = g.nseg - 1;
    if (g.glu) return "gemm_dma_glu";
    if (g.nseg > 1 && g.seg[last].rows <= 64 && g.seg_start[last] % 64 == 0)
      return g.seg[last].is_i8 || g.seg[last].rows / 16 > (g.N - g.seg[last].rows + 255) / 256
                 ? "gemm_dma+lora_skinny"
                 : "gemm_dma+lora";
    return "gemm_dma";
  }
  if (g.glu) return "gemm_skinny_glu";
  bool i8 = false;
  for (int i = 0; i < g.nseg; ++i) i8 = i8 || g.seg[i].is_i8;
  if ((g.M / 16) % 8 == 0 && !i8 && !g.rowstats && skinny_ok(g.M, g.N, g.K) &&
      g.split <= g.K / 64)
    return "gemm_skinny";
  return "gemm_nt";
}

hipError_t gemm_nt(const GemmArgs& g, hipStream_t st) {
  if (g.M <= 0 || g.N <= 0 || g.M % 16 || g.K % KSTEP || g.K < KSTEP || g.split < 1 ||
      g.split > g.K / KSTEP || g.nseg < 1 || g.nseg > 4) {
    set_error("gemm_nt: unsupported shape M=%d N=%d K=%d split=%d", g.M, g.N, g.K, g.split);
    return hipErrorInvalidValue;
  }
  for (int i = 0; i < g.nseg; ++i)
    if (g.seg[i].rows % 16) {
      set_error("gemm_nt: segment rows must be a multiple of 16 (%d)", g.seg[i].rows);
      return hipErrorInvalidValue;
    }
  if (g.glu && !(g.N == 2 * g.glu && g.nseg == 1 && g.split == 1 && g.glu16 && g.gu16 &&
                 gemm_glu_ok(g.M, g.glu, g.K, g.seg[0].is_i8))) {
    set_error("gemm_nt: SwiGLU epilogue needs split 1, one segment, N = 2 x %d", g.glu);
    return hipErrorInvalidValue;
  }
  if (g.split_col && !use_big_tiles(g)) {
    set_error("gemm_nt: split_col needs the large-tile kernel");
    return hipErrorInvalidValue;
  }
  if (g.rowstats && gemm_rowstats_tiles(g) == 0) {
    set_error("gemm_nt: row statistics need split 1, one segment and no SwiGLU epilogue");
    return hipErrorInvalidValue;
  }
  if (g.glu && !use_big_tiles(g)) {
    hipLaunchKernelGGL((gemm_skinny_kernel<4, 4, true>), dim3(1, g.glu / 32, g.M / 128), dim3(512),
                       0, st, g);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) set_error("gemm_nt launch: %s", hipGetErrorString(e));
    return e;
  }
  hipError_t e;
  const int m16 = g.M / 16;
  if (use_big_tiles(g)) {
    GemmArgs gm = g;
    const int last = g.nseg - 1;
    const bool lora_tail = g.nseg > 1 && g.seg[last].rows <= 64 && g.seg_start[last] % 64 == 0;
    if (lora_tail) {  // the main segments on big tiles, the LoRA rows skinny
      gm.nseg = last;
      gemm_finalize_segments(gm);
    }
    const int nwg = (gm.N + 255) / 256 * (gm.M / BM);
    // XCD-contiguous tile runs: workgroup b goes to XCD b % 8, and the tiles
    // sharing an A row block then share that XCD's L2 (C4: +0.7% step rate)
    const int order = 1;
    const bool i8 = gm.seg[0].is_i8, ks = gm.seg[0].kscale != nullptr;
    if (gm.nseg != 1 || gm.N % 16 != 0) {
      set_error("gemm_nt: large tiles take one B segment with N %% 16 == 0 (N = %d, %d segments)",
                gm.N, gm.nseg);
      return hipErrorInvalidValue;
    }
    if (gm.split_col > 0 &&
        (gm.split != 2 || gm.split_col % 256 || gm.split_col >= gm.N || gm.N % 256 || gm.glu ||
         gm.rowstats || lora_tail)) {
      set_error("gemm_nt: split_col %d needs split 2 and whole 256-column tiles (N = %d)",
                gm.split_col, gm.N);
      return hipErrorInvalidValue;
    }
    const dim3 gr = gm.split_col > 0
                        ? dim3(gm.split_col / 256 * (gm.M / BM) + 2 * (gm.N - gm.split_col) / 256 * (gm.M / BM), 1)
                        : dim3(nwg, gm.split);
    // the LoRA rows fold into the main launch (fragment f with column tile f)
    // when they are fp16 and no more fragments than column tiles
    const BSeg tl = lora_tail ? g.seg[last] : BSeg{};
    const bool fold = lora_tail && !tl.is_i8 && tl.rows / 16 <= (gm.N + 255) / 256;
    const int tc0 = lora_tail ? g.seg_start[last] : 0;
    // ring depth 5 (int8) / 4 (fp16): 4 measured the same, 6 slower
    auto go = [&](auto i8c, auto ksc, auto gluc, auto tlc) {
      constexpr bool I8 = decltype(i8c)::value, KS = decltype(ksc)::value;
      constexpr bool GL = decltype(gluc)::value, TLc = decltype(tlc)::value;
      constexpr int SD = I8 ? 5 : 4;
      hipLaunchKernelGGL((gemm_dma_kernel<I8, KS, SD, 4, GL, TLc>), gr, dim3(512), 0, st, gm, order,
                         tl, tc0);
    };
    using BT = std::integral_constant<bool, true>;
    using BF = std::integral_constant<bool, false>;
    if (gm.glu) {
      if (!i8) go(BF(), BF(), BT(), BF());
      else if (ks) go(BT(), BT(), BT(), BF());
      else go(BT(), BF(), BT(), BF());
    } else if (fold) {
      if (!i8) go(BF(), BF(), BF(), BT());
      else if (ks) go(BT(), BT(), BF(), BT());
      else go(BT(), BF(), BF(), BT());
    } else {
      if (!i8) go(BF(), BF(), BF(), BF());
      else if (ks) go(BT(), BT(), BF(), BF());
      else go(BT(), BF(), BF(), BF());
    }
    e = hipGetLastError();
    if (e == hipSuccess && lora_tail && !fold) {
      GemmArgs gl = g;
      gl.nseg = 1;
      gl.seg[0] = g.seg[last];
      gemm_finalize_segments(gl);
      gl.C = g.C + g.seg_start[last];
      e = launch_m128(gl, st);
    }
  } else if (m16 % 8 == 0) e = launch_m128(g, st);
  else if (m16 % 4 == 0) e = launch_mf<4>(g, st);
  else if (m16 % 2 == 0) e = launch_mf<2>(g, st);
  else e = launch_mf<1>(g, st);
  if (e != hipSuccess) set_error("gemm_nt launch: %s", hipGetErrorString(e));
  return e;
}

hipError_t reduce_lora(const ReduceArgs& a, hipStream_t st) {
  if (a.M % 16 || a.N % 4 || a.ldp % 4 || a.ldo % 4 || a.nlora < 0 || a.nlora > 3 ||
      a.out == a.part) {
    set_error("reduce_lora: M %% 16, N/ldp/ldo %% 4, nlora <= 3 and out != part required");
    return hipErrorInvalidValue;
  }
  for (int q = 0; q < a.nlora; ++q)
    if (a.up[q].c0 % 64 || a.up[q].n % 64 || a.up[q].hcol % 4) {
      set_error("reduce_lora: adapter column ranges must be 64-aligned, h columns 4-aligned");
      return hipErrorInvalidValue;
    }
  dim3 grid((a.N + 63) / 64, a.M / 16);
  hipLaunchKernelGGL(reduce_lora_kernel, grid, dim3(256), 0, st, a);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t pack_f16(const _Float16* src, long long lds, int transpose, int R, int C, _Float16* dst,
                    long long K, int row0, int k0, hipStream_t st) {
  if (C % 8 || k0 % 8 || K % 32) {
    set_error("pack_f16: C, k0 must be multiples of 8 and K of 32");
    return hipErrorInvalidValue;
  }
  const long long np = (long long)R * (C / 8);
  hipLaunchKernelGGL(pack_kernel<_Float16>, dim3(grid1d(np, 256)), dim3(256), 0, st, src, lds,
                     transpose, R, C, dst, K, row0, k0, nullptr);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t pack_i8(const int8_t* src, long long lds, int transpose, int R, int C, int8_t* dst,
                   long long K, int row0, int k0, hipStream_t st, const _Float16* zs) {
  if (C % 8 || k0 % 8 || K % 32) {
    set_error("pack_i8: C, k0 must be multiples of 8 and K of 32");
    return hipErrorInvalidValue;
  }
  const long long np = (long long)R * (C / 8);
  hipLaunchKernelGGL(pack_kernel<int8_t>, dim3(grid1d(np, 256)), dim3(256), 0, st, src, lds,
                     transpose, R, C, dst, K, row0, k0, zs);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t transpose_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  hipLaunchKernelGGL(transpose_f16_kernel, grid, dim3(256), 0, st, src, rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t transpose_i8(const int8_t* src, int rows, int cols, int lds, int8_t* dst, int ldd,
                        hipStream_t st) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  hipLaunchKernelGGL(transpose_i8_kernel, grid, dim3(256), 0, st, src, rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f32_to_f16(const float* src, _Float16* dst, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(f32_to_f16_kernel, dim3(grid1d(n, 256)), dim3(256), 0, st, src, dst, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t copy_rows_f16(const _Float16* src, int rows, int cols, int lds, _Float16* dst, int ldd,
                         hipStream_t st) {
  const long long n = (long long)rows * cols;
  hipLaunchKernelGGL(copy_rows_f16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, src,
                     rows, cols, lds, dst, ldd);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t fill_f32(float* dst, float v, size_t n, hipStream_t st) {
  hipLaunchKernelGGL(fill_f32_kernel, dim3(grid1d(n, 256)), dim3(256), 0, st, dst, v, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t quantize_rows_i8(const float* w, int rows, int cols, int8_t* q, float* scale,
                            hipStream_t st) {
  hipLaunchKernelGGL(quantize_rows_kernel, dim3(rows), dim3(256), 0, st, w, cols, q, scale);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

hipError_t f32_scale_to_f16(const float* s, _Float16* d, int n, hipStream_t st) {
  hipLaunchKernelGGL(f32_scale_to_f16_kernel, dim3((n + 255) / 256), dim3(256), 0, st, s, d, n);
  LLMT_LAUNCH_CHECK();
  return hipSuccess;
}

}  // namespace llmt
