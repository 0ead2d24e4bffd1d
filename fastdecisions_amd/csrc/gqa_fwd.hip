// Native GQA causal attention forward for gfx950 (bf16 MFMA, fp32 softmax).
//
// Computes what the reference's Triton kernel computes
// (ref: src/decider/native_gqa_kernel.py:6-113): per query head h, kv head
// h / (Hq/Hkv) (:39-41); S = Q K^T * scale; causal mask key <= query (:63-81);
// online softmax with running max / denominator and correction
// exp(m_old - m_new) (:84-104); P rounded to bf16 before P·V (:98-102);
// out = acc / denominator (:106-113).  The design is CDNA4's own:
//
// * One workgroup = the query heads of one KV group x 32 queries; for
//   head_dim <= 128 it has 8 wavefronts, two per SIMD: the two wavefronts of a
//   head split every 64-key tile into its two 32-key halves (each keeps its
//   own running max / denominator / accumulator; they are merged through LDS
//   at the end).  Two wavefronts per SIMD let one run softmax VALU work while
//   the other issues MFMAs.  head_dim 256 runs 4 wavefronts (register budget).
// * K and V tiles (64 keys) are copied global -> LDS with global_load_lds
//   (no staging registers, no VALU), one barrier per tile.  For head_dim
//   <= 128 the ring has 4 stages and the loop is software-pipelined: while a
//   wavefront finishes tile t (mask, softmax, P·V), the scores of tile t+1
//   are computed, one MFMA of that dependent chain after each of eight pieces
//   of the softmax, so the VALU work issues while the MFMAs run; tiles t+2 and
//   t+3 are in flight.
// * head_dim 256: one wavefront per head (4 per workgroup), each walking
//   32-key blocks; the P·V of block j-1 and the scores of block j+1 are
//   issued with the softmax of block j between their MFMAs, over 2-stage K
//   and V rings.
// * Which loop runs depends on head_dim alone, so for head_dim <= 128 a
//   request's output rows are bit-identical whether it runs alone, packed
//   with others (cu_seqlens) or in a padded batch of any size.
//   16-byte chunks are XOR-swizzled per row so that the MFMA operand reads
//   below are bank-conflict free.
// * The score tile is computed transposed, S^T = K · Q^T, with
//   v_mfma_f32_32x32x16_bf16.  In the 32x32 accumulator a lane owns one
//   column (= one query) and 16 rows (= keys), so the softmax row max and sum
//   are lane-local except for one exchange between the two lane halves
//   (v_permlane32_swap).
// * The K rows fed to the MFMA are permuted (sigma below) so that the 8 keys a
//   lane holds for each 16-key slice of P are exactly the 8 consecutive keys
//   it must supply as the B operand of O^T += V^T · P^T: P never leaves
//   registers.  The V^T A operand comes straight from the row-major V tile
//   with two ds_read_b64_tr_b16 (transposing LDS reads) per MFMA.
// * The output is accumulated transposed (O^T), so the per-query rescale and
//   the final 1/denominator are lane-local.  The scale is folded into the exp2
//   argument (one fma per score), masks run only on diagonal / tail tiles, and
//   the running max is raised lazily (only when a tile exceeds it by more than
//   2^8), so the O rescale is skipped on most tiles.
// * Work items are ordered longest-first (causal tiles near the end of the
//   sequence have the most keys) and mapped so that each XCD receives a
//   contiguous range of (head group, query tile) items, keeping a KV head's
//   tiles in one L2.
#include <algorithm>
#include <type_traits>

#include "fd_common.h"

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));

namespace {

constexpr int kBlockM = 32;  // queries per wavefront
constexpr int kBlockN = 64;  // keys per LDS tile
constexpr int kNumXcd = 8;
constexpr int kMaxUnits = 768;  // work units per group of a split launch (kernel-argument table)

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;

// The fields the work-item decode reads come first: a workgroup's first
// scalar loads of its arguments then share cache lines.
struct GqaArgs {
  int n_items;    // work items (workgroups with work)
  int n_qtiles;   // query tiles per (sequence, head group)
  int n_hgroups;  // q_heads / hpw
  int hpw;        // query heads per workgroup
  int qpw;        // 32-query blocks per workgroup (hpw * qpw == 4)
  int q_heads, kv_heads, seq_len;
  // Key split of the long query tiles (padded batches with fewer work items
  // than CUs): the n_split longest tiles of every (sequence, head group) run as
  // two items over the two halves of their key tiles, each writing its
  // unnormalised (o, running max, denominator) to `part`; gqa_combine_kernel
  // merges them.
  int n_split;    // 0: no split
  int n_groups;   // sequences * head groups
  int n_units;    // work units per group: n_qtiles + n_split
  int n_pad;      // n_units rounded up to a multiple of xcd_per_group
  int xcd_per_group;
  float scale_log2;
  const int32_t* cu;
  int n_seqs;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t qs[4], ks[4], vs[4], os[4];
  const uint16_t* gate;  // output gate (fd_gqa_gated_fwd) or null
  int64_t gs[4];
  float* part;    // [n_groups][n_split][2][4 slots][64 lanes][D/2 + 4]: o, max, denominator, 2 pad
  // units of a group, longest first: 4 * query tile + (part + 1), part -1 = whole tile
  uint16_t units[kMaxUnits];
};

// KSPLIT = wavefronts per (head, query block): each takes 64/KSPLIT keys of a tile.
template <int D, int KSPLIT>
struct Cfg {
  static constexpr int kWaves = 4 * KSPLIT;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kBlocks = 2 / KSPLIT;                 // 32-key blocks per wavefront per tile
  static constexpr int kChunksRow = D / 8;                   // 16-byte chunks per K / V row
  static constexpr int kTileBytes = kBlockN * kChunksRow * 16;
  static constexpr int kLoads = kBlockN * kChunksRow / kThreads;  // global_load_lds per thread per K (or V) tile
  static constexpr int kStageBytes = 2 * kTileBytes;         // K tile + V tile
  // Pipelined loop (two wavefronts per (head, query block) and 4 stages in
  // LDS): the scores of tile t+1 are computed while tile t is finished, and
  // tiles t+2, t+3 are in flight.  head_dim 256 (one wavefront per (head,
  // query block)) has 2 stages, used as separate K and V rings.
  static constexpr bool kPipe = KSPLIT > 1 && 4 * kStageBytes <= 160 * 1024;
  static constexpr int kStages = kPipe ? 4 : 2;
  // merge of the key parts: half an O, the running max and the denominator from each
  static constexpr int kCombineBytes = KSPLIT > 1 ? 8 * 64 * (D / 4 + 2) * 4 : 0;
  static constexpr int kSmemBytes =
      (kStages * kStageBytes > kCombineBytes) ? kStages * kStageBytes : kCombineBytes;
  // s_waitcnt immediate: vmcnt(N) with expcnt / lgkmcnt left alone (gfx9 encoding)
  static constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
  static_assert(kLoads * kThreads == kBlockN * kChunksRow, "tile must split evenly over the threads");
};

// Key (within a 32-key block) supplied by MFMA row m, chosen so that the
// accumulator registers 8j..8j+7 of lane half g hold keys 16j + 8g + 0..7.
__device__ __forceinline__ int sigma(int m) {
  return ((m >> 4) << 4) + (((m >> 2) & 1) << 3) + (((m >> 3) & 1) << 2) + (m & 3);
}

// Chunk swizzles (physical chunk = logical chunk ^ f(row)).  K: the MFMA A
// operand reads rows sigma(0..7) = {0,1,2,3,8,9,10,11} (then +4) at one chunk;
// a bit permutation of row & 15 sends any 8 of them to 8 distinct chunks.
// V: 16 lanes of a transposing read touch 4 consecutive rows x 2 adjacent
// chunks, 32 lanes 4 rows x 4 chunks; the xor keeps chunk pairs adjacent.
template <int CR>
__device__ __forceinline__ int swz_k(int row) {
  const int r = row & 15;
  return ((r & 3) | ((r & 8) >> 1) | ((r & 4) << 1)) & (CR - 1);
}
template <int CR>
__device__ __forceinline__ int swz_v(int row) {
  // 16+ chunks per row: xor with 4*(row & 3) puts the 4 rows x 4 chunks that
  // 32 lanes of a transposing read touch on 16 distinct chunks (all banks).
  return CR >= 16 ? 4 * (row & 3) : (2 * (row & 3)) & (CR - 1);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

// Max / sum of a value over lanes l and l^32 (the two lane halves hold the two
// 16-key halves of one query's scores).  v_permlane32_swap with the value in
// both operands leaves this lane's value in one result and its partner's in
// the other, so max and sum of the pair need no lane-index select.
__device__ __forceinline__ float half_max(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_sum(float v) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Floats per lane record of a split tile's half in the workspace: O^T (D/2),
// running max, denominator and two pad floats, so every record (and each of
// its 16-byte vector accesses) is 16-byte aligned.
template <int D>
constexpr int kPartFloats = D / 2 + 4;

// Workspace slot of one (head, query block) slot x lane of a split tile's half.
template <int D>
__device__ __forceinline__ float* part_slot(const GqaArgs& a, int group, int qtile, int part, int w4, int lane) {
  const size_t tile = static_cast<size_t>(group) * a.n_split + (a.n_qtiles - 1 - qtile);
  return a.part + ((tile * 2 + part) * 4 * 64 + w4 * 64 + lane) * kPartFloats<D>;
}

// Normalised store of a lane's query row (the O^T accumulator: dims
// 32 db + 8 r4 + 4 half + 0..3) for the O blocks [DB0, DB1), with the optional
// output gate bf16(o) * bf16(sigmoid(gate)), each product rounded to bf16 as
// the eager ops do.  The gate loads all go out before the first is used.
template <int D, int DB0 = 0, int DB1 = D / 32>
__device__ __forceinline__ void store_rows(const GqaArgs& a, const f32x16_t (&o)[D / 32], float inv, bool qvalid,
                                           uint16_t* orow, const uint16_t* grow, int half) {
  if (!qvalid) return;
  bf16x4_t gb[DB1 - DB0][4];
  if (grow != nullptr) {
#pragma unroll
    for (int db = DB0; db < DB1; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        gb[db - DB0][r4] = *reinterpret_cast<const bf16x4_t*>(grow + db * 32 + r4 * 8 + half * 4);
  }
#pragma unroll
  for (int db = DB0; db < DB1; ++db) {
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int d = db * 32 + r4 * 8 + half * 4;
      f32x4_t v4 = {o[db][r4 * 4 + 0] * inv, o[db][r4 * 4 + 1] * inv, o[db][r4 * 4 + 2] * inv,
                    o[db][r4 * 4 + 3] * inv};
      bf16x4_t ob = __builtin_convertvector(v4, bf16x4_t);
      if (grow != nullptr) {
        const f32x4_t gf = __builtin_convertvector(gb[db - DB0][r4], f32x4_t);
        const f32x4_t of = __builtin_convertvector(ob, f32x4_t);
        f32x4_t sg, pr;
#pragma unroll
        for (int e = 0; e < 4; ++e) sg[e] = 1.0f / (1.0f + expf(-gf[e]));
        const f32x4_t sgr = __builtin_convertvector(__builtin_convertvector(sg, bf16x4_t), f32x4_t);
#pragma unroll
        for (int e = 0; e < 4; ++e) pr[e] = of[e] * sgr[e];
        ob = __builtin_convertvector(pr, bf16x4_t);
      }
      *reinterpret_cast<bf16x4_t*>(orow + d) = ob;
    }
  }
}

template <int D, int KSPLIT>
__global__ __launch_bounds__(256 * KSPLIT, 1) void gqa_fwd_kernel(GqaArgs a) {
  using C = Cfg<D, KSPLIT>;
  constexpr int CR = C::kChunksRow;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[C::kSmemBytes];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: copy destinations stay scalar
  const int w4 = wave & 3;     // (head, query block) slot
  const int kh = wave >> 2;    // key part of each tile (0 when KSPLIT == 1)
  const int col = lane & 31;   // query within the wavefront's block
  const int half = lane >> 5;

  // ---- work item
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  int qtile, wgroup, part = -1;
  if (a.n_split > 0) {
    // Key split.  Block b runs on XCD b % 8; each group (one KV head's query
    // heads of one sequence) goes to xcd_per_group XCDs, which take every
    // xcd_per_group-th unit of its longest-first list in turn: each XCD's L2
    // holds one KV head, and every XCD gets an equal share of long and short
    // units, started longest first.
    const int L = (b % kNumXcd) * (nb / kNumXcd) + b / kNumXcd;
    wgroup = L / a.n_pad;
    const int p = L % a.n_pad;
    const int chunk = a.n_pad / a.xcd_per_group;
    const int u = __builtin_amdgcn_readfirstlane((p % chunk) * a.xcd_per_group + p / chunk);
    if (wgroup >= a.n_groups || u >= a.n_units) return;
    const int code = a.units[u];  // uniform index: a scalar load
    qtile = code >> 2;
    part = (code & 3) - 1;
  } else {
    // XCD-contiguous renumbering, longest tile first
    const int item = (nb % kNumXcd == 0) ? (b % kNumXcd) * (nb / kNumXcd) + b / kNumXcd : b;
    if (item >= a.n_items) return;
    qtile = a.n_qtiles - 1 - item % a.n_qtiles;
    wgroup = item / a.n_qtiles;
  }
  const int hg = wgroup % a.n_hgroups;
  const int sidx = wgroup / a.n_hgroups;

  int seq_start, seq_end, bidx;
  if (a.cu != nullptr) {
    // clamped to [0, T], so a malformed offset table cannot move an access outside q/k/v/o
    seq_start = min(max(a.cu[sidx], 0), a.seq_len);
    seq_end = min(max(a.cu[sidx + 1], seq_start), a.seq_len);
    bidx = 0;
  } else {
    seq_start = 0;
    seq_end = a.seq_len;
    bidx = sidx;
  }
  const int qspan = kBlockM * a.qpw;
  const int q0 = seq_start + qtile * qspan;
  if (q0 >= seq_end) return;  // uniform over the workgroup

  const int group = a.q_heads / a.kv_heads;
  const int hsub = w4 % a.hpw;
  const int qb = w4 / a.hpw;
  const int qhead = hg * a.hpw + hsub;
  const int kvhead = (hg * a.hpw) / group;

  const uint16_t* qbase = a.q + bidx * a.qs[0] + qhead * a.qs[1];
  const uint16_t* kbase = a.k + bidx * a.ks[0] + kvhead * a.ks[1];
  const uint16_t* vbase = a.v + bidx * a.vs[0] + kvhead * a.vs[1];
  uint16_t* obase = a.o + bidx * a.os[0] + qhead * a.os[1];

  const int qw0 = q0 + qb * kBlockM;  // first query of this wavefront
  const int qpos = qw0 + col;
  const bool qvalid = qpos < seq_end;
  const float c = a.scale_log2;

  // Q^T as MFMA B operand: lane supplies Q[qpos][16kk + 8*half + 0..7].
  bf16x8_t qf[D / 16];
  if constexpr (KSPLIT == 1) {
    // The head_dim-256 loop issues its copies and LDS reads as asm and counts
    // them itself; the compiler, which does not see them, must not be left
    // with loads of its own to wait for inside the loop.  So Q is read with
    // asm too, before any copy, and the prologue's copy wait covers it.  Rows
    // past the end read the last row and are zeroed after that wait.
    typedef unsigned u32x4q_t __attribute__((ext_vector_type(4)));
    const int qrow = qvalid ? qpos : seq_end - 1;
    const uint16_t* qp = qbase + qrow * a.qs[2] + half * 8;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      u32x4q_t raw;
      asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(raw) : "v"(qp), "i"(kk * 32) : "memory");
      qf[kk] = __builtin_bit_cast(bf16x8_t, raw);
    }
  } else {
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      uint4 u = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) u = *reinterpret_cast<const uint4*>(qbase + qpos * a.qs[2] + kk * 16 + half * 8);
      qf[kk] = as_bf16x8(u);
    }
  }

  const int kend = min(q0 + qspan, seq_end);
  const int nt_all = (kend - seq_start + kBlockN - 1) / kBlockN;
  // key tiles [tb, tb + ntiles) of this item (a half of them for a split tile)
  const int tb = part == 1 ? nt_all / 2 : 0;
  const int ntiles = part == 0 ? nt_all / 2 : nt_all - tb;

  // ---- per-lane addressing, computed once.  LDS: [K stage 0..S-1][V stage
  // 0..S-1]; K and V reads each use one base register plus an immediate
  // stage offset (< 64 KiB), the loop being unrolled by the stage count.
  unsigned char* const k_lds = smem;
  unsigned char* const v_lds = smem + C::kStages * C::kTileBytes;
  // global -> LDS copies: copy i of this lane moves 16-byte chunk `slot` of a
  // tile (row = slot / CR, physical chunk = slot % CR, global chunk unswizzled)
  auto cp_row = [&](int i) { return ((i * C::kWaves + wave) * 64 + lane) / CR; };
  auto cp_koff = [&](int i) {
    const int slot = (i * C::kWaves + wave) * 64 + lane;
    return ((slot % CR) ^ swz_k<CR>(slot / CR)) * 8;
  };
  auto cp_voff = [&](int i) {
    const int slot = (i * C::kWaves + wave) * 64 + lane;
    return ((slot % CR) ^ swz_v<CR>(slot / CR)) * 8;
  };
  // K A operand: lane reads row (kh*kBlocks + bl)*32 + sigma(col), logical chunk 2kk + half.
  // V^T A operand: two transposing reads per (dim block, 16-key slice).
  // With two wavefronts per SIMD the byte offsets fit in registers and are
  // computed once; the 4-wavefront head_dim-256 variant recomputes them.
  const int grp = lane >> 4;
  const int li = lane & 15;
  auto k_off_calc = [&](int bl, int kk) {
    const int row = (kh * C::kBlocks + bl) * 32 + sigma(col);
    return row * CR * 16 + (((2 * kk + half) ^ swz_k<CR>(row)) * 16);
  };
  auto v_off_calc = [&](int db, int cs, int r2) {
    const int dim = db * 32 + 16 * (grp & 1) + 4 * (li & 3);
    const int row = ((kh * C::kBlocks) * 2 + cs) * 16 + 8 * (grp >> 1) + 4 * r2 + (li >> 2);
    return row * CR * 16 + (((dim >> 3) ^ swz_v<CR>(row)) * 16) + (dim & 7) * 2;
  };
  constexpr bool kHoist = KSPLIT > 1;
  int k_rd[kHoist ? C::kBlocks : 1][kHoist ? D / 16 : 1];
  int v_rd[kHoist ? D / 32 : 1][kHoist ? 2 * C::kBlocks : 1][2];
  if constexpr (kHoist) {
#pragma unroll
    for (int bl = 0; bl < C::kBlocks; ++bl)
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) k_rd[bl][kk] = k_off_calc(bl, kk);
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int cs = 0; cs < 2 * C::kBlocks; ++cs)
#pragma unroll
        for (int r2 = 0; r2 < 2; ++r2) v_rd[db][cs][r2] = C::kStages * C::kTileBytes + v_off_calc(db, cs, r2);
  }
  int cp_krel[kHoist ? C::kLoads : 1], cp_vrel[kHoist ? C::kLoads : 1];
  if constexpr (kHoist) {
#pragma unroll
    for (int i = 0; i < C::kLoads; ++i) {
      cp_krel[i] = cp_row(i) * static_cast<int>(a.ks[2]) + cp_koff(i);
      cp_vrel[i] = cp_row(i) * static_cast<int>(a.vs[2]) + cp_voff(i);
    }
  }
  auto k_off = [&](int bl, int kk) {
    if constexpr (kHoist) return k_rd[bl][kk]; else return k_off_calc(bl, kk);
  };
  // V^T operand address in stage BUF: the hoisted offsets include the V region's
  // base, so the stage offset (< 64 KiB) is the read's immediate
  auto v_addr = [&](int BUF, int db, int cs, int r2) -> const unsigned char* {
    if constexpr (kHoist) return smem + BUF * C::kTileBytes + v_rd[db][cs][r2];
    else return v_lds + BUF * C::kTileBytes + v_off_calc(db, cs, r2);
  };

  // rows past the end of the sequence re-read its last row: finite data the mask discards
  auto issue_tile = [&](int t, int buf) {
    const int ks0 = seq_start + (tb + t) * kBlockN;
    unsigned char* kt = k_lds + buf * C::kTileBytes;
    unsigned char* vt = v_lds + buf * C::kTileBytes;
    const uint16_t* kg = kbase + ks0 * a.ks[2];
    const uint16_t* vg = vbase + ks0 * a.vs[2];
    const bool full = ks0 + kBlockN <= seq_end;
    const int last = seq_end - 1 - ks0;  // last valid row of this tile
#pragma unroll
    for (int i = 0; i < C::kLoads; ++i) {
      const int blk = i * C::kWaves + wave;
      int krel, vrel;
      if (full) {
        krel = kHoist ? cp_krel[i] : cp_row(i) * static_cast<int>(a.ks[2]) + cp_koff(i);
        vrel = kHoist ? cp_vrel[i] : cp_row(i) * static_cast<int>(a.vs[2]) + cp_voff(i);
      } else {
        const int r = cp_row(i) < last ? cp_row(i) : last;
        krel = r * static_cast<int>(a.ks[2]) + cp_koff(i);
        vrel = r * static_cast<int>(a.vs[2]) + cp_voff(i);
      }
      // uniform tile base + 32-bit per-lane byte offset (scalar-base addressing)
      const void* ksrc = reinterpret_cast<const unsigned char*>(kg) + static_cast<uint32_t>(krel) * 2u;
      const void* vsrc = reinterpret_cast<const unsigned char*>(vg) + static_cast<uint32_t>(vrel) * 2u;
      __builtin_amdgcn_global_load_lds(ksrc, (lds_void_t*)(kt + blk * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vsrc, (lds_void_t*)(vt + blk * 1024), 16, 0, 0);
    }
  };

  f32x16_t o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db) o[db] = f32x16_t{};
  float m_run = -__builtin_inff();  // running max (log2-scaled units), may lag the true max by <= 8
  float l_run = 0.0f;               // this lane's partial denominator

  constexpr int kPerTile = 2 * C::kLoads;  // VMEM instructions per thread of one issue_tile

  // S^T for this wavefront's 32-key block(s) of the tile in LDS stage BUF
  auto scores = [&](int BUF, f32x16_t (&s)[C::kBlocks]) {
    const unsigned char* kt = k_lds + BUF * C::kTileBytes;
#pragma unroll
    for (int bl = 0; bl < C::kBlocks; ++bl) {
      s[bl] = f32x16_t{};
      constexpr int kGroup = D / 16 < 8 ? D / 16 : 8;  // operand reads issued ahead of their MFMAs
#pragma unroll
      for (int k0 = 0; k0 < D / 16; k0 += kGroup) {
        bf16x8_t kf[kGroup];
#pragma unroll
        for (int kk = 0; kk < kGroup; ++kk) kf[kk] = *reinterpret_cast<const bf16x8_t*>(kt + k_off(bl, k0 + kk));
#pragma unroll
        for (int kk = 0; kk < kGroup; ++kk)
          s[bl] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[k0 + kk], s[bl], 0, 0, 0);
      }
    }
  };

  // causal / end-of-sequence mask of tile t, on diagonal and tail tiles only
  auto mask = [&](int t, f32x16_t (&s)[C::kBlocks]) {
    const int kb0 = seq_start + (tb + t) * kBlockN + kh * C::kBlocks * 32;  // first key of this wavefront's part
    if (kb0 + C::kBlocks * 32 - 1 > qw0 || kb0 + C::kBlocks * 32 > seq_end) {
#pragma unroll
      for (int bl = 0; bl < C::kBlocks; ++bl)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb0 + bl * 32 + (r >> 3) * 16 + half * 8 + (r & 7);
          if (key > qpos || key >= seq_end) s[bl][r] = -__builtin_inff();
        }
    }
  };

  // O = alpha O + V^T · P^T with V in stage BUF: the V^T A operand of each
  // 16-key slice comes from two transposing reads of the row-major V tile
  // (keys +0..3 and +4..7)
  auto accumulate = [&](int BUF, const bf16x8_t (&pb)[2 * C::kBlocks], float alpha, bool grow_any) {
    if (grow_any) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
    }
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
#pragma unroll
      for (int cs = 0; cs < 2 * C::kBlocks; ++cs) {
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)v_addr(BUF, db, cs, 0));
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t*)v_addr(BUF, db, cs, 1));
        const short __attribute__((ext_vector_type(8))) vv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), pb[cs], o[db], 0, 0, 0);
      }
    }
  };

  if constexpr (C::kPipe) {
    // Prologue: tiles 0..2 in flight, wait for tiles 0 and 1, scores of tile 0.
    issue_tile(0, 0);
    if (ntiles > 1) issue_tile(1, 1);
    if (ntiles > 2) {
      issue_tile(2, 2);
      __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(kPerTile));
    } else {
      __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(0));
    }
    __syncthreads();
    f32x16_t sA[C::kBlocks], sB[C::kBlocks];
    scores(0, sA);

    // Step t (stage BUF = t % 4): tile t+3 is issued into the stage tile t-1
    // left (every wavefront passed the previous step's barrier); the softmax
    // of tile t and the scores of tile t+1 (complete since the previous step)
    // are independent, so their VALU and MFMA work can interleave.  At the
    // end only tile t+3 may still be in flight: tile t+2, which the next
    // step's scores read, has landed, and the barrier makes it visible.  The
    // last step's scores read a stale stage and are discarded.
    auto step = [&](int t, int BUF, f32x16_t (&sc)[C::kBlocks], f32x16_t (&sn)[C::kBlocks]) {
      static_assert(C::kBlocks == 1, "the pipelined step takes one 32-key block per wavefront");
      const bool issued = t + 3 < ntiles;
      if (issued) issue_tile(t + 3, (BUF + 3) & 3);
      mask(t, sc);
      // The next tile's scores are a chain of D/16 dependent MFMAs; after each
      // one the wavefront issues one piece of this tile's softmax (8 pieces),
      // which runs while the MFMA does.  sched_barrier keeps the pieces apart.
      constexpr int kSteps = D / 16;
      constexpr int kPer = 8 / kSteps;  // softmax pieces per MFMA
      const unsigned char* ktn = k_lds + ((BUF + 1) & 3) * C::kTileBytes;
      float mx = -__builtin_inff(), alpha = 1.0f, m_sub = 0.0f, psum = 0.0f;
      bool grow = false;
      f32x8_t pv[2];
      bf16x8_t pb[2];
      auto piece = [&](int k) {
        if (k == 0) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[0][r]);
        } else if (k == 1) {
          mx = half_max(mx) * c;
          grow = mx > m_run + 8.0f;
          const float m_new = grow ? mx : m_run;
          alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
          m_sub = (m_new == -__builtin_inff()) ? 0.0f : m_new;  // fully masked so far: p = 0
          m_run = m_new;
        } else if (k < 6) {
          const int r0 = 4 * (k - 2);  // scores r0 .. r0 + 3
#pragma unroll
          for (int r = r0; r < r0 + 4; ++r) {
            float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[0][r], c, -m_sub));
            asm volatile("" : "+v"(p));  // computed here, not sunk towards its use in P·V
            psum += p;
            pv[r >> 3][r & 7] = p;
          }
        } else if (k == 6) {
          pb[0] = __builtin_convertvector(pv[0], bf16x8_t);
          pb[1] = __builtin_convertvector(pv[1], bf16x8_t);
          asm volatile("" : "+v"(pb[0]), "+v"(pb[1]));
        } else {
          l_run = l_run * alpha + psum;
          asm volatile("" : "+v"(l_run));
        }
      };
      // All of the next tile's K operands are read before the chain: the
      // compiler then waits once per tile for them (read one MFMA ahead, it
      // waited at every MFMA for the read just issued); 38.6 -> 38.1 us at B=1.
      sn[0] = f32x16_t{};
      bf16x8_t kfa[kSteps];
#pragma unroll
      for (int kk = 0; kk < kSteps; ++kk) kfa[kk] = *reinterpret_cast<const bf16x8_t*>(ktn + k_off(0, kk));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < kSteps; ++kk) {
        sn[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kfa[kk], qf[kk], sn[0], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < kPer; ++j) piece(kk * kPer + j);
        __builtin_amdgcn_sched_barrier(0);
      }
      const bool grow_any = __builtin_amdgcn_ballot_w64(grow) != 0;
      accumulate(BUF, pb, alpha, grow_any);
      if (issued)
        __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(kPerTile));
      else
        __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(0));
      __syncthreads();
    };
    int t = 0;
    for (; t + 4 <= ntiles; t += 4) {
      step(t, 0, sA, sB);
      step(t + 1, 1, sB, sA);
      step(t + 2, 2, sA, sB);
      step(t + 3, 3, sB, sA);
    }
    if (t < ntiles) step(t, 0, sA, sB);
    if (t + 1 < ntiles) step(t + 1, 1, sB, sA);
    if (t + 2 < ntiles) step(t + 2, 2, sA, sB);
  } else if constexpr (KSPLIT == 1) {
    // head_dim 256: one wavefront per SIMD (4 per workgroup), each owning one
    // head's 32 queries.  The wavefront walks the keys in 32-key blocks (block
    // b = half b % 2 of tile b / 2) with its own online softmax per block.
    // Block step j issues the 16 P·V MFMAs of block j-1 and the 16 score MFMAs
    // of block j+1 alternately, and between them the softmax of block j, so
    // the VALU work runs under the MFMAs.  K and V have 2-stage rings of whole
    // tiles: K(u) is copied in step 2u-3 and read in steps 2u-1, 2u; V(u) is
    // copied in step 2u-1 and read in steps 2u+1, 2u+2.  Copies and LDS
    // operand reads are asm with explicit waits (see the Q loads).
    constexpr int kKk = D / 16;   // score MFMAs per block (and P·V MFMAs)
    constexpr int kNdb = D / 32;  // O^T blocks
    constexpr int RB = CR * 16;   // bytes per K / V row in LDS
    constexpr int kRowsPer = 64 / CR;  // rows per 1 KiB copy instruction
    constexpr int kKPer = 16 / (4 * kRowsPer) > 1 ? 16 / (4 * kRowsPer) : 1;  // period of the K copy swizzle in i
    constexpr int kPieceEvery = kKk >= 8 ? kKk / 8 : 1;  // MFMA pairs per softmax piece
    constexpr int kPiecesPer = kKk >= 8 ? 1 : 8 / kKk;    // softmax pieces per MFMA pair
    constexpr int kWin = 4;       // MFMA pairs (three reads each) in flight
    static_assert(C::kBlocks == 2 && C::kStages == 2, "one-wavefront-per-head layout");
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)smem));
    // copy offsets: slot (i*4 + wave)*64 + lane -> row 8i + 2 wave + lane/32, chunk lane%32;
    // the K swizzle depends on row & 15, i.e. on i & 1
    const int crow = kRowsPer * wave + lane / CR;
    const int cchunk = lane % CR;
    int ck_off[kKPer];
#pragma unroll
    for (int e = 0; e < kKPer; ++e) ck_off[e] = (cchunk ^ swz_k<CR>(4 * kRowsPer * e + crow)) * 8;
    const int cv_off = (cchunk ^ swz_v<CR>(crow)) * 8;
    auto copy_tile = [&](int u, bool is_v) {
      const uint32_t stage_base = lds0 + static_cast<uint32_t>(((is_v ? 2 : 0) + (u & 1)) * C::kTileBytes);
      const int ks0 = seq_start + (tb + u) * kBlockN;
      const uint16_t* g = is_v ? vbase + ks0 * a.vs[2] : kbase + ks0 * a.ks[2];
      const int stride = static_cast<int>(is_v ? a.vs[2] : a.ks[2]);
      const int last = seq_end - 1 - ks0;  // rows past the end re-read the last row: finite data the mask discards
#pragma unroll
      for (int i = 0; i < C::kLoads; ++i) {
        const int r = min(4 * kRowsPer * i + crow, last);
        const int rel = r * stride + (is_v ? cv_off : ck_off[i % kKPer]);
        const uint32_t lds = stage_base + static_cast<uint32_t>((i * C::kWaves + wave) * 1024);
        asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                     :: "v"(static_cast<uint32_t>(rel) * 2u), "s"(g), "s"(lds) : "memory", "m0");
      }
    };
    // K operand (block bl of a tile, step kk): row bl*32 + sigma(col), logical chunk 2kk + half;
    // chunk (16 hi + lo) ^ z = 16 hi + (lo ^ z): 8 lane offsets, the rest immediates
    const int krow = sigma(col);
    const int kz = swz_k<CR>(krow);
    constexpr int kNkq = kKk < 8 ? kKk : 8;
    uint32_t kq[kNkq];
#pragma unroll
    for (int k3 = 0; k3 < kNkq; ++k3) kq[k3] = lds0 + static_cast<uint32_t>(krow * RB + (((2 * k3 + half) ^ kz) * 16));
    // V^T operand (O block db = 4 dh + d2, 16-key slice cs of the tile, half r2):
    // row 16 cs + 8 (grp >> 1) + 4 r2 + li / 4, chunk 16 dh + 4 (d2 ^ (li / 4 & 3)) + c0
    const int vrow = 8 * (grp >> 1) + (li >> 2);
    const int vc0 = 2 * (grp & 1) + ((li & 3) >> 1);
    constexpr int kNvq = kNdb < 4 ? kNdb : 4;
    uint32_t vq[kNvq];
#pragma unroll
    for (int d2 = 0; d2 < kNvq; ++d2)
      vq[d2] = lds0 + static_cast<uint32_t>(2 * C::kTileBytes + vrow * RB + (((4 * d2 + vc0) ^ swz_v<CR>(vrow)) * 16) + 8 * (li & 1));
    typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
    const int nblk = 2 * ntiles;

    // causal / end-of-sequence mask of block b, on diagonal and tail blocks only
    auto mask_block = [&](int b, f32x16_t& s) {
      const int kb0 = seq_start + tb * kBlockN + b * 32;
      if (kb0 + 31 > qw0 || kb0 + 32 > seq_end) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb0 + (r >> 3) * 16 + half * 8 + (r & 7);
          if (key > qpos || key >= seq_end) s[r] = -__builtin_inff();
        }
      }
    };

    // prologue: K0, K1, V0 in flight; scores of block 0 once K0 has landed
    copy_tile(0, false);
    if (ntiles > 1) copy_tile(1, false);
    copy_tile(0, true);
    if (ntiles > 1) __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(2 * C::kLoads));
    else __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(C::kLoads));
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {  // the Q loads (older than every copy) have completed
      asm volatile("" : "+v"(qf[kk]));
      if (!qvalid) qf[kk] = bf16x8_t{};
    }
    __syncthreads();
    f32x16_t S[2];   // scores of block b in S[b & 1]
    bf16x8_t P[2][2];  // P of block b in P[b & 1] (two 16-key slices)
    S[0] = f32x16_t{};
    {
      u32x4_t kf0[kWin];
#define FD_R0(I) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kf0[(I) % kWin]) \
                              : "v"(kq[(I) % kNkq]), "i"(256 * ((I) / kNkq)) : "memory")
#pragma unroll
      for (int kk = 0; kk < kWin && kk < kKk; ++kk) FD_R0(kk);
#pragma unroll
      for (int kk = 0; kk < kKk; ++kk) {
        const int younger = min(kWin - 1, kKk - 1 - kk);
#define FD_W0(N) asm volatile("s_waitcnt lgkmcnt(" #N ")" : "+v"(kf0[kk % kWin]) :: "memory")
        switch (younger) {
          case 3: FD_W0(3); break;
          case 2: FD_W0(2); break;
          case 1: FD_W0(1); break;
          default: FD_W0(0); break;
        }
#undef FD_W0
        S[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf0[kk % kWin]), qf[kk], S[0], 0, 0, 0);
        if (kk + kWin < kKk) FD_R0(kk + kWin);
        __builtin_amdgcn_sched_barrier(0);
      }
#undef FD_R0
    }

    // block step j: P·V of block j-1 (PV), softmax of block j (SM), scores of
    // block j+1 (SC).  PAR = j & 1 picks the score and P registers; the LDS
    // stage and half-tile offsets are added to the lane offsets once per step.
    auto step = [&](auto PAR_C, auto PV_C, auto SM_C, auto SC_C, int j) {
      constexpr int PAR = decltype(PAR_C)::value;
      constexpr bool PV = decltype(PV_C)::value, SM = decltype(SM_C)::value, SC = decltype(SC_C)::value;
      f32x16_t& ssm = S[PAR];             // block j
      f32x16_t& ssc = S[PAR ^ 1];         // block j+1
      bf16x8_t (&ppv)[2] = P[PAR ^ 1];    // block j-1
      bf16x8_t (&psm)[2] = P[PAR];        // block j
      // K of block j+1: tile (j+1)/2 in stage ((j+1)/2) & 1, half (j+1) & 1;
      // V of block j-1: tile (j-1)/2, half (j-1) & 1 (its 16-key slices 2 half, 2 half + 1)
      const uint32_t koff = static_cast<uint32_t>((((j + 1) >> 1) & 1) * C::kTileBytes + ((j + 1) & 1) * 32 * RB);
      const uint32_t voff = static_cast<uint32_t>((((j - 1) >> 1) & 1) * C::kTileBytes + ((j - 1) & 1) * 32 * RB);
      uint32_t kqs[kNkq], vqs[kNvq];
      if constexpr (SC) {
#pragma unroll
        for (int k3 = 0; k3 < kNkq; ++k3) kqs[k3] = kq[k3] + koff;
      }
      if constexpr (PV) {
#pragma unroll
        for (int d2 = 0; d2 < kNvq; ++d2) vqs[d2] = vq[d2] + voff;
      }
      if (PAR == 1) {  // odd steps copy K((j+3)/2) and V((j+1)/2)
        const int uk = (j + 3) >> 1, uv = (j + 1) >> 1;
        if (uk < ntiles) copy_tile(uk, false);
        if (uv < ntiles) copy_tile(uv, true);
      }
      float mx = -__builtin_inff(), alpha = 1.0f, m_sub = 0.0f, psum = 0.0f;
      bool grow = false;
      f32x8_t pv8[2];
      auto piece = [&](int k) {
        if constexpr (SM) {
          if (k == 0) {
            mask_block(j, ssm);
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, ssm[r]);
          } else if (k == 1) {
            mx = half_max(mx) * c;
            grow = mx > m_run + 8.0f;
            const float m_new = grow ? mx : m_run;
            alpha = grow ? __builtin_amdgcn_exp2f(m_run - m_new) : 1.0f;
            m_sub = (m_new == -__builtin_inff()) ? 0.0f : m_new;  // fully masked so far: p = 0
            m_run = m_new;
          } else if (k < 6) {
            const int r0 = 4 * (k - 2);
#pragma unroll
            for (int r = r0; r < r0 + 4; ++r) {
              float p = __builtin_amdgcn_exp2f(__builtin_fmaf(ssm[r], c, -m_sub));
              asm volatile("" : "+v"(p));
              psum += p;
              pv8[r >> 3][r & 7] = p;
            }
          } else if (k == 6) {
            psm[0] = __builtin_convertvector(pv8[0], bf16x8_t);
            psm[1] = __builtin_convertvector(pv8[1], bf16x8_t);
            asm volatile("" : "+v"(psm[0]), "+v"(psm[1]));
          } else if (k == 7) {
            l_run = l_run * alpha + psum;
            asm volatile("" : "+v"(l_run));
          }
        }
      };
      if constexpr (PV || SC) {
        constexpr int per = (SC ? 1 : 0) + (PV ? 2 : 0);
        u32x4_t kf[kWin];
        u32x2_t vlo[kWin], vhi[kWin];
        // pair i: score MFMA step kk = i, P·V MFMA m = i (O block m & 7, slice m >> 3)
#define FD_R(I)                                                                                                 \
  do {                                                                                                          \
    const int i_ = (I), w_ = i_ % kWin;                                                                         \
    if constexpr (SC)                                                                                           \
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kf[w_]) : "v"(kqs[i_ % kNkq]), "i"(256 * (i_ / kNkq)) \
                   : "memory");                                                                                 \
    if constexpr (PV) {                                                                                         \
      const int db_ = i_ % kNdb, cs_ = i_ / kNdb;                                                               \
      asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(vlo[w_])                                        \
                   : "v"(vqs[db_ % kNvq]), "i"(256 * (db_ / kNvq) + 16 * RB * cs_) : "memory");                 \
      asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(vhi[w_])                                        \
                   : "v"(vqs[db_ % kNvq]), "i"(256 * (db_ / kNvq) + 16 * RB * cs_ + 4 * RB) : "memory");        \
    }                                                                                                           \
  } while (0)
#pragma unroll
        for (int i = 0; i < kWin; ++i) FD_R(i);
        if constexpr (SC) ssc = f32x16_t{};
#pragma unroll
        for (int i = 0; i < kKk; ++i) {
          const int w = i % kWin;
          const int younger = per * min(kWin - 1, kKk - 1 - i);
#define FD_W(N) asm volatile("s_waitcnt lgkmcnt(" #N ")" : "+v"(kf[w]), "+v"(vlo[w]), "+v"(vhi[w]) :: "memory")
          switch (younger) {
            case 12: FD_W(12); break;
            case 9: FD_W(9); break;
            case 8: FD_W(8); break;
            case 6: FD_W(6); break;
            case 4: FD_W(4); break;
            case 3: FD_W(3); break;
            case 2: FD_W(2); break;
            case 1: FD_W(1); break;
            default: FD_W(0); break;
          }
#undef FD_W
          if constexpr (SC)
            ssc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[w]), qf[i], ssc, 0, 0, 0);
          if constexpr (PV) {
            const u32x4_t vv = {vlo[w][0], vlo[w][1], vhi[w][0], vhi[w][1]};
            o[i % kNdb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), ppv[i / kNdb], o[i % kNdb], 0, 0, 0);
          }
          if (i % kPieceEvery == kPieceEvery - 1) {
#pragma unroll
            for (int pp = 0; pp < kPiecesPer; ++pp) piece((i / kPieceEvery) * kPiecesPer + pp);
          }
          if (i + kWin < kKk) FD_R(i + kWin);
          __builtin_amdgcn_sched_barrier(0);
        }
#undef FD_R
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) piece(k);
      }
      if constexpr (SM) {
        // O is relative to the running max from here on (after this step's P·V)
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
          for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
        }
      }
      // the next step reads K of block j+2 and V of block j: even steps wait for
      // every copy, odd ones for all but their own
      if (PAR == 0) {
        __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(0));
      } else {
        const int own = ((((j + 3) >> 1) < ntiles) ? C::kLoads : 0) + ((((j + 1) >> 1) < ntiles) ? C::kLoads : 0);
        if (own >= 2 * C::kLoads) __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(2 * C::kLoads));
        else if (own >= C::kLoads) __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(C::kLoads));
        else __builtin_amdgcn_s_waitcnt(C::waitcnt_vm(0));
      }
      __syncthreads();
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // step 0 (no P·V yet); steady steps 1 .. nblk-2 (an even count); step
    // nblk-1 (no scores); step nblk (the last P·V).  nblk = 2 ntiles is even.
    step(I0{}, F_{}, T_{}, T_{}, 0);
    for (int j = 1; j + 2 < nblk; j += 2) {
      step(I1{}, T_{}, T_{}, T_{}, j);
      step(I0{}, T_{}, T_{}, T_{}, j + 1);
    }
    step(I1{}, T_{}, T_{}, F_{}, nblk - 1);
    step(I0{}, T_{}, F_{}, F_{}, nblk);
  } else {
    static_assert(C::kPipe || KSPLIT == 1, "no loop for this configuration");
  }

  // ---- merge the key parts of each (head, query block), then normalise and store
  uint16_t* const orow = obase + qpos * a.os[2];
  const uint16_t* const grow = a.gate ? a.gate + bidx * a.gs[0] + qhead * a.gs[1] + qpos * a.gs[2] : nullptr;
  if constexpr (KSPLIT > 1) {
    // (head_dim <= 128 never splits a tile over workgroups, so every item is a
    // whole tile.)  Each key part hands the other the half of O it does not store and
    // finishes the half it does (kh 0: blocks 0 .. D/64-1, kh 1: the rest),
    // so both wavefronts of a SIMD run the normalisation, gate and store.
    // Every element is the same sum of the same two products as a one-sided
    // merge gives.
    constexpr int kHalf = D / 64;          // O blocks per half
    constexpr int kStride = kHalf * 16 + 2;  // floats per lane: the half, max, denominator
    float* const mine = reinterpret_cast<float*>(smem) + ((kh * 4 + w4) * 64 + lane) * kStride;
    const float* const theirs = reinterpret_cast<const float*>(smem) + (((kh ^ 1) * 4 + w4) * 64 + lane) * kStride;
    // KEEP: the first O block this key part stores (compile-time, so that o
    // stays in registers)
    auto hand_over = [&](auto keep_c) {
      constexpr int GIVE = kHalf - decltype(keep_c)::value;
#pragma unroll
      for (int b = 0; b < kHalf; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) mine[b * 16 + r] = o[GIVE + b][r];
      mine[kHalf * 16] = m_run;
      mine[kHalf * 16 + 1] = l_run;
    };
    auto finish = [&](auto keep_c) {
      constexpr int KEEP = decltype(keep_c)::value;
      const float m1 = theirs[kHalf * 16];
      const float l1 = theirs[kHalf * 16 + 1];
      const float m = fmaxf(m_run, m1);
      const float a0 = (m_run == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m_run - m);
      const float a1 = (m1 == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
      const float l_tot = half_sum(l_run * a0 + l1 * a1);
#pragma unroll
      for (int b = 0; b < kHalf; ++b)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[KEEP + b][r] = o[KEEP + b][r] * a0 + theirs[b * 16 + r] * a1;
      store_rows<D, KEEP, KEEP + kHalf>(a, o, 1.0f / l_tot, qvalid, orow, grow, half);
    };
    using Lo = std::integral_constant<int, 0>;
    using Hi = std::integral_constant<int, kHalf>;
    if (kh == 0) hand_over(Lo{});
    else hand_over(Hi{});
    __syncthreads();
    if (kh == 0) finish(Lo{});
    else finish(Hi{});
    return;
  }
  if (part >= 0) {
    // a half of a split tile: the unnormalised state goes to the workspace
    float* dst = part_slot<D>(a, wgroup, qtile, part, w4, lane);
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4)
        *reinterpret_cast<f32x4_t*>(dst + db * 16 + r4 * 4) =
            f32x4_t{o[db][r4 * 4], o[db][r4 * 4 + 1], o[db][r4 * 4 + 2], o[db][r4 * 4 + 3]};
    dst[D / 2] = m_run;
    dst[D / 2 + 1] = l_run;
    return;
  }
  const float l_tot = half_sum(l_run);
  store_rows<D>(a, o, 1.0f / l_tot, qvalid, orow, grow, half);
}

// Merge of the two halves of every split tile (one wavefront per tile and
// (head, query block) slot, lanes as in the main kernel): the same combine as
// the in-workgroup merge of the key parts, then the normalised, optionally
// gated store.
template <int D>
__global__ __launch_bounds__(64) void gqa_combine_kernel(GqaArgs a) {
  const int lane = threadIdx.x;
  const int w4 = blockIdx.x % 4;  // one wavefront per (split tile, slot): every CU takes a share
  const int tile = blockIdx.x / 4;
  const int group = tile / a.n_split;
  const int qtile = a.n_qtiles - 1 - tile % a.n_split;
  const int hg = group % a.n_hgroups;
  const int bidx = group / a.n_hgroups;  // split tiles are padded batches only (no cu_seqlens)
  const int qhead = hg * a.hpw + w4 % a.hpw;
  const int qpos = qtile * kBlockM * a.qpw + (w4 / a.hpw) * kBlockM + (lane & 31);
  const float* p0 = part_slot<D>(a, group, qtile, 0, w4, lane);
  const float* p1 = part_slot<D>(a, group, qtile, 1, w4, lane);
  const float m0 = p0[D / 2], l0 = p0[D / 2 + 1];
  const float m1 = p1[D / 2], l1 = p1[D / 2 + 1];
  const float m = fmaxf(m0, m1);
  const float a0 = (m0 == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m0 - m);
  const float a1 = (m1 == -__builtin_inff()) ? 0.0f : __builtin_amdgcn_exp2f(m1 - m);
  f32x16_t o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const f32x4_t x0 = *reinterpret_cast<const f32x4_t*>(p0 + db * 16 + r4 * 4);
      const f32x4_t x1 = *reinterpret_cast<const f32x4_t*>(p1 + db * 16 + r4 * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[db][r4 * 4 + e] = x0[e] * a0 + x1[e] * a1;
    }
  const float l_tot = half_sum(l0 * a0 + l1 * a1);
  const bool qvalid = qpos < a.seq_len;
  store_rows<D>(a, o, 1.0f / l_tot, qvalid, a.o + bidx * a.os[0] + qhead * a.os[1] + qpos * a.os[2],
                a.gate ? a.gate + bidx * a.gs[0] + qhead * a.gs[1] + qpos * a.gs[2] : nullptr, lane >> 5);
}

int gcd_int(int x, int y) {
  while (y) {
    int t = x % y;
    x = y;
    y = t;
  }
  return x;
}

bool stride_ok(const int64_t s[4]) {
  if (s[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if (s[i] % 8 != 0) return false;  // 16-byte rows
  return true;
}

// Key split (head_dim 256 only): a padded batch with fewer work items than
// the 256 CUs of the MI355X (e.g. B=1, T=2048, 8/2 heads of 256: 128 items)
// runs the longest half of its query tiles as two items over the two halves
// of their key tiles, merged by gqa_combine_kernel.  The merge rounds
// differently from the whole-tile loop, so a head_dim-256 row depends on
// whether the split ran (the caller turns it off by passing no workspace).
// head_dim 64 and 128 never split: at one item per CU (B=1, T=2048, 16/4
// heads of 128) the split measured no faster, and without it every launch of
// these head dims runs the same loop, whatever the batch.
constexpr int64_t kSplitBelow = 256;

// Query tiles of every (sequence, head group) that the key split halves, or 0.
int split_tiles(int n_qtiles, int64_t items, bool varlen, int head_dim) {
  if (head_dim != 256 || varlen || items >= kSplitBelow || n_qtiles < 4 || n_qtiles + n_qtiles / 2 > kMaxUnits)
    return 0;
  return n_qtiles / 2;
}

// The unit table of a split launch: whole tiles and halves of the n_split
// longest, sorted by their key-tile count, longest first (the diagonal half
// of a tile before the other), and the XCD sharing of the groups.
void fill_units(GqaArgs& a, int qspan) {
  struct U {
    int len, code;
  };
  U list[kMaxUnits];
  int n = 0;
  for (int t = a.n_qtiles - 1; t >= 0; --t) {
    const int nt = (std::min((t + 1) * qspan, a.seq_len) + kBlockN - 1) / kBlockN;
    if (t >= a.n_qtiles - a.n_split) {
      list[n++] = U{nt - nt / 2, 4 * t + 2};  // part 1: key tiles [nt/2, nt)
      list[n++] = U{nt / 2, 4 * t + 1};       // part 0: key tiles [0, nt/2)
    } else {
      list[n++] = U{nt, 4 * t};
    }
  }
  std::stable_sort(list, list + n, [](const U& x, const U& y) { return x.len > y.len; });
  for (int i = 0; i < n; ++i) a.units[i] = static_cast<uint16_t>(list[i].code);
  a.n_units = n;
  a.xcd_per_group = (a.n_groups < kNumXcd && kNumXcd % a.n_groups == 0) ? kNumXcd / a.n_groups : 1;
  a.n_pad = (n + a.xcd_per_group - 1) / a.xcd_per_group * a.xcd_per_group;
}

int64_t split_bytes(int64_t n_groups, int n_split, int head_dim) {
  return n_groups * n_split * 2 * 4 * 64 * static_cast<int64_t>(head_dim / 2 + 4) * 4;
}

// Sizes shared by the launcher and fd_gqa_workspace_bytes.
struct GqaShape {
  int hpw, qpw, n_qtiles, n_hgroups, n_slots;
  int64_t items;
};
GqaShape gqa_shape(int batch, int q_heads, int kv_heads, int seq_len, int n_seqs, int max_seqlen, bool varlen) {
  GqaShape g;
  const int group = q_heads / kv_heads;
  g.hpw = gcd_int(group, 4);
  g.qpw = 4 / g.hpw;
  const int span_len = varlen ? max_seqlen : seq_len;
  g.n_slots = varlen ? n_seqs : batch;
  g.n_qtiles = (span_len + kBlockM * g.qpw - 1) / (kBlockM * g.qpw);
  g.n_hgroups = q_heads / g.hpw;
  g.items = static_cast<int64_t>(g.n_qtiles) * g.n_hgroups * g.n_slots;
  return g;
}

int gqa_launch(const void* q, const void* k, const void* v, void* out, const int64_t q_strides[4],
               const int64_t k_strides[4], const int64_t v_strides[4], const int64_t out_strides[4],
               const void* gate, const int64_t gate_strides[4], int batch, int q_heads, int kv_heads, int seq_len,
               int head_dim, float scale, const int32_t* cu_seqlens, int n_seqs, int max_seqlen, void* workspace,
               int64_t workspace_bytes, void* stream) {
  FD_REQUIRE(q && k && v && out && q_strides && k_strides && v_strides && out_strides, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: tensor and stride pointers must be non-null");
  FD_REQUIRE(batch >= 0 && seq_len >= 0 && q_heads >= 1 && kv_heads >= 1, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: batch/seq_len must be >= 0 and head counts >= 1");
  FD_REQUIRE(q_heads % kv_heads == 0, FD_ERR_INVALID_ARGUMENT,
             "fd_gqa_fwd: q_heads (%d) must be divisible by kv_heads (%d)", q_heads, kv_heads);
  FD_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, FD_ERR_UNSUPPORTED,
             "fd_gqa_fwd: head_dim must be 64, 128 or 256 (got %d)", head_dim);
  FD_REQUIRE(scale > 0.0f && scale < 1e30f, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: scale must be positive");
  FD_REQUIRE(stride_ok(q_strides) && stride_ok(k_strides) && stride_ok(v_strides) && stride_ok(out_strides),
             FD_ERR_ALIGNMENT,
             "fd_gqa_fwd: innermost strides must be 1 and the others multiples of 8 elements (16 bytes)");
  FD_REQUIRE(fd_aligned16(q) && fd_aligned16(k) && fd_aligned16(v) && fd_aligned16(out), FD_ERR_ALIGNMENT,
             "fd_gqa_fwd: tensors must be 16-byte aligned");
  // K/V tile rows are addressed with 32-bit offsets from the tile's first row
  FD_REQUIRE(k_strides[2] >= 0 && v_strides[2] >= 0 && k_strides[2] < (1 << 24) && v_strides[2] < (1 << 24),
             FD_ERR_UNSUPPORTED, "fd_gqa_fwd: K/V token strides must be in [0, 2^24) elements");
  int n_slots;
  int span_len;
  if (cu_seqlens != nullptr) {
    FD_REQUIRE(batch == 1, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: cu_seqlens requires batch == 1 (got %d)", batch);
    FD_REQUIRE(n_seqs >= 1, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: n_seqs must be >= 1");
    FD_REQUIRE(max_seqlen >= 0 && max_seqlen <= seq_len, FD_ERR_INVALID_ARGUMENT,
               "fd_gqa_fwd: max_seqlen must be in [0, seq_len]");
    n_slots = n_seqs;
    span_len = max_seqlen;
  } else {
    n_slots = batch;
    span_len = seq_len;
  }
  if (n_slots == 0 || span_len == 0) return FD_OK;

  const GqaShape g = gqa_shape(batch, q_heads, kv_heads, seq_len, n_seqs, max_seqlen, cu_seqlens != nullptr);
  GqaArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.o = static_cast<uint16_t*>(out);
  a.gate = static_cast<const uint16_t*>(gate);
  for (int i = 0; i < 4; ++i) a.gs[i] = gate ? gate_strides[i] : 0;
  for (int i = 0; i < 4; ++i) {
    a.qs[i] = q_strides[i];
    a.ks[i] = k_strides[i];
    a.vs[i] = v_strides[i];
    a.os[i] = out_strides[i];
  }
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.seq_len = seq_len;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.cu = cu_seqlens;
  a.n_seqs = n_seqs;
  a.hpw = g.hpw;
  a.qpw = g.qpw;
  a.n_qtiles = g.n_qtiles;
  a.n_hgroups = g.n_hgroups;
  FD_REQUIRE(g.items < 2147483647LL / 2, FD_ERR_INVALID_ARGUMENT, "fd_gqa_fwd: problem too large");
  a.n_groups = g.n_hgroups * g.n_slots;
  a.n_split = split_tiles(g.n_qtiles, g.items, cu_seqlens != nullptr, head_dim);
  a.part = static_cast<float*>(workspace);
  if (a.n_split > 0 && (workspace == nullptr || !fd_aligned16(workspace) ||
                        workspace_bytes < split_bytes(a.n_groups, a.n_split, head_dim)))
    a.n_split = 0;  // no room for the halves: every tile runs whole
  int64_t items = g.items;
  if (a.n_split > 0) {
    fill_units(a, kBlockM * g.qpw);
    items = static_cast<int64_t>(a.n_groups) * a.n_pad;
  }
  a.n_items = static_cast<int>(items);
  const int nblocks = static_cast<int>((items + kNumXcd - 1) / kNumXcd * kNumXcd);
  hipStream_t s = static_cast<hipStream_t>(stream);
  dim3 grid(nblocks);
  switch (head_dim) {
    case 64:
      hipLaunchKernelGGL((gqa_fwd_kernel<64, 2>), grid, dim3(Cfg<64, 2>::kThreads), 0, s, a);
      break;
    case 128:
      hipLaunchKernelGGL((gqa_fwd_kernel<128, 2>), grid, dim3(Cfg<128, 2>::kThreads), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((gqa_fwd_kernel<256, 1>), grid, dim3(Cfg<256, 1>::kThreads), 0, s, a);
      break;
  }
  if (a.n_split > 0) {
    const dim3 cgrid(static_cast<unsigned>(a.n_groups * a.n_split * 4));
    hipLaunchKernelGGL(gqa_combine_kernel<256>, cgrid, dim3(64), 0, s, a);
  }
  return fd_check_launch("fd_gqa_fwd");
}

}  // namespace

extern "C" int fd_gqa_fwd(const void* q, const void* k, const void* v, void* out, const int64_t q_strides[4],
                          const int64_t k_strides[4], const int64_t v_strides[4], const int64_t out_strides[4],
                          int batch, int q_heads, int kv_heads, int seq_len, int head_dim, float scale,
                          const int32_t* cu_seqlens, int n_seqs, int max_seqlen, void* workspace,
                          int64_t workspace_bytes, void* stream) {
  return gqa_launch(q, k, v, out, q_strides, k_strides, v_strides, out_strides, nullptr, nullptr, batch, q_heads,
                    kv_heads, seq_len, head_dim, scale, cu_seqlens, n_seqs, max_seqlen, workspace, workspace_bytes,
                    stream);
}

extern "C" int fd_gqa_gated_fwd(const void* q, const void* k, const void* v, const void* gate, void* out,
                                const int64_t q_strides[4], const int64_t k_strides[4], const int64_t v_strides[4],
                                const int64_t gate_strides[4], const int64_t out_strides[4], int batch,
                                int q_heads, int kv_heads, int seq_len, int head_dim, float scale,
                                const int32_t* cu_seqlens, int n_seqs, int max_seqlen, void* workspace,
                                int64_t workspace_bytes, void* stream) {
  FD_REQUIRE(gate && gate_strides, FD_ERR_INVALID_ARGUMENT, "fd_gqa_gated_fwd: gate and its strides must be non-null");
  FD_REQUIRE(fd_aligned16(gate) && gate_strides[3] == 1 && gate_strides[0] % 8 == 0 && gate_strides[1] % 8 == 0 &&
                 gate_strides[2] % 8 == 0,
             FD_ERR_ALIGNMENT, "fd_gqa_gated_fwd: gate must keep 16-byte rows with a unit innermost stride");
  return gqa_launch(q, k, v, out, q_strides, k_strides, v_strides, out_strides, gate, gate_strides, batch, q_heads,
                    kv_heads, seq_len, head_dim, scale, cu_seqlens, n_seqs, max_seqlen, workspace, workspace_bytes,
                    stream);
}

extern "C" int64_t fd_gqa_workspace_bytes(int batch, int q_heads, int kv_heads, int seq_len, int head_dim,
                                          int n_seqs, int max_seqlen) {
  if (batch < 0 || seq_len < 0 || q_heads < 1 || kv_heads < 1 || q_heads % kv_heads != 0) return FD_ERR_INVALID_ARGUMENT;
  if (head_dim != 64 && head_dim != 128 && head_dim != 256) return FD_ERR_UNSUPPORTED;
  const bool varlen = n_seqs > 0;
  if (varlen && (batch != 1 || max_seqlen < 0 || max_seqlen > seq_len)) return FD_ERR_INVALID_ARGUMENT;
  const GqaShape g = gqa_shape(batch, q_heads, kv_heads, seq_len, n_seqs, max_seqlen, varlen);
  const int n_split = split_tiles(g.n_qtiles, g.items, varlen, head_dim);
  return n_split > 0 ? split_bytes(static_cast<int64_t>(g.n_hgroups) * g.n_slots, n_split, head_dim) : 0;
}
