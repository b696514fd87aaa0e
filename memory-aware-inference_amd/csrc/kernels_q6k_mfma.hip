// Q6_K matvec on the gfx950 matrix cores (replaces si_q6_k_matvec* for one
// input vector, src/metal.rs:895-1081; the output head of the greedy decode
// and the MLP down projection).
//
// Weights.  quant.rs:145-171 decodes half h (128 elements) of a block from
// ql[64h .. 64h + 64), qh[32h .. 32h + 32) and scales[8h .. 8h + 8): element
// 128h + 32t + l (t = 0..3, l = 0..31) is (6-bit q) - 32 with scale
// 8h + 2t + l / 16.  Lane group g = 2h + s of the B operand owns l in
// [16s, 16s + 16) of half h for all four t: its 16-byte pieces are ql at
// 64h + 16s (low nibbles: t = 0, high: t = 2), ql at 64h + 32 + 16s (t = 1, 3)
// and qh at 128 + 32h + 16s (two bits per t), and MFMA t of a block gets one
// scale per lane.  The MFMA takes the unsigned q (0..63); a second MFMA of the
// same image with every weight byte -32 adds the offset, so each lane's digit
// sums C_t[d] = sum (q - 32) D_d are exact integers.
//
// Per block and lane: T_d = sum_t sc_t * C_t[d] in integers, y += d * (sum_d
// T_d * 256^d) * 2^(e_b - 30) (the digit images of the activations are built
// as for Q4_K, mfma_common.h).  A block with side elements is a rounded
// block, whose rows recompute it exactly when its error bound fails the
// rounded-block check (mfma_common.h); blocks whose activations are not
// finite or reach 2^100 take the exact per-weight f32 path whole
// (w = (d * sc) * (q - 32), quant.rs rounding).
//
// Data path.  Blocks are 210 bytes, so they are not 16-byte aligned; with an
// even block count nb every row and every stage of two blocks (420 bytes)
// starts on a 4-byte boundary, which the 16-byte buffer->LDS copies need (odd
// nb runs as row pairs, PAIRED below).  Each row's 420 bytes of a stage arrive
// with 27 copies in piece-major order, piece q of row r at LDS byte
// 16 (16 q + r), so every read is a conflict-free 16-lane sweep.  Pieces 0..25
// are bytes 16 q .. 16 q + 15; piece 26 is bytes 404..419, so no copy runs
// past the stage (a copy that crosses the end of its buffer descriptor reads
// as zero in full).  The second block of a stage starts 2 bytes into piece
// 13: its chunks are read as two pieces and realigned with v_alignbyte.
// Scheduling, the LDS slot ring and the finishing wave are the Q4_K
// kernel's (mfma_common.h).
#include "argmax_device.h"
#include "mfma_common.h"
#include "si_hip_tuned.h"
#include "tokens_common.h"

namespace sihip {
namespace {

using namespace mfma;

constexpr uint32_t kStageRowBytes = 2u * kQ6Bytes;     // 420: two blocks of one row
constexpr uint32_t kRowPieces = 27u;                   // pieces per row and stage
constexpr uint32_t kLastPiece = kStageRowBytes - 16u;  // 404: start of piece 26
constexpr uint32_t kCopies = 7u;                       // 7 x 64 lanes >= 16 rows x 27 pieces
constexpr uint32_t kStageBytes = kCopies * 1024u;      // 7168
static_assert(16u * (kRowPieces - 1u) <= kStageRowBytes && kLastPiece % 4u == 0u,
              "pieces 0..25 and 26 lie inside the stage, 4-byte aligned");
static_assert(16u * kRowPieces <= kCopies * 64u, "copies cover every piece");

__host__ __device__ constexpr Layout layout(uint32_t waves, uint32_t depth, uint32_t nb,
                                            uint32_t slots, uint32_t ntok = 1u,
                                            uint32_t sums = 1u) {
  return make_layout(kStageBytes, 2u, 0u, waves, depth, nb, slots, sums, ntok);
}

// The lane's 13 pieces of a stage buffer (piece q of row n at 256 q + 16 n;
// qa = piece 4h + s, qh = piece 8 + 2h + s, sc = piece 12 of the lane's row):
//   v0 ql chunk A, v1 ql chunk B (piece +2), v2 qh chunk, v3 scales,
//   v4 piece 13 (d of block 0) -- block 0;
//   v5,v6 / v7,v8 / v9,v10 the same chunks of block 1 (13 pieces later, two
//   pieces each), v11 piece 25 (stage bytes 400..415), v12 piece 26 (bytes
//   404..419) -- its scales and d, block 1.
__device__ __forceinline__ void lds_read_stage(uint32_t qa, uint32_t qh, uint32_t sc,
                                               u32x4 (&v)[13]) {
  asm volatile(
      "ds_read_b128 %0, %13\n"
      "ds_read_b128 %1, %13 offset:512\n"
      "ds_read_b128 %2, %14\n"
      "ds_read_b128 %3, %15\n"
      "ds_read_b128 %4, %15 offset:256\n"
      "ds_read_b128 %5, %13 offset:3328\n"
      "ds_read_b128 %6, %13 offset:3584\n"
      "ds_read_b128 %7, %13 offset:3840\n"
      "ds_read_b128 %8, %13 offset:4096\n"
      "ds_read_b128 %9, %14 offset:3328\n"
      "ds_read_b128 %10, %14 offset:3584\n"
      "ds_read_b128 %11, %15 offset:3328\n"
      "ds_read_b128 %12, %15 offset:3584\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
        "=&v"(v[12])
      : "v"(qa), "v"(qh), "v"(sc)
      : "memory");
}

// The 8 A images of a stage (block b, MFMA t at addr + 1024 b + 256 t), read
// only by the lanes in `mask`; the other lanes keep their (zero) registers.
__device__ __forceinline__ void lds_read_images(uint32_t addr, uint64_t mask, i32x4 (&a)[8]) {
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %[sv], exec\n"
      "s_mov_b64 exec, %[m]\n"
      "ds_read_b128 %0, %[ad]\n"
      "ds_read_b128 %1, %[ad] offset:256\n"
      "ds_read_b128 %2, %[ad] offset:512\n"
      "ds_read_b128 %3, %[ad] offset:768\n"
      "ds_read_b128 %4, %[ad] offset:1024\n"
      "ds_read_b128 %5, %[ad] offset:1280\n"
      "ds_read_b128 %6, %[ad] offset:1536\n"
      "ds_read_b128 %7, %[ad] offset:1792\n"
      "s_waitcnt lgkmcnt(0)\n"
      "s_mov_b64 exec, %[sv]"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]),
        "+v"(a[7]), [sv] "=&s"(saved)
      : [ad] "v"(addr), [m] "s"(mask)
      : "memory");
}

// The stage's two block exponents (ea) and their side counts (one byte
// each, at ea + kCountOff).
__device__ __forceinline__ void lds_read_expo(uint32_t ea, u32x2& ex, uint32_t& cnt) {
  static_assert(kCountOff == 512, "the offset below");
  asm volatile(
      "ds_read_b64 %0, %2\n"
      "ds_read_u16 %1, %2 offset:512\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(ex), "=&v"(cnt)
      : "v"(ea)
      : "memory");
}

// Signed byte of w at bit offset `bit` (an int8 scale).
__device__ __forceinline__ int scale_at(uint32_t w, uint32_t bit) {
  return (int)__builtin_amdgcn_sbfe((int)w, bit, 8u);
}

// The 16 bytes that start 2 bytes into piece lo (and end in piece hi).
__device__ __forceinline__ u32x4 skip2(const u32x4& lo, const u32x4& hi) {
  return u32x4{__builtin_amdgcn_alignbyte(lo[1], lo[0], 2), __builtin_amdgcn_alignbyte(lo[2], lo[1], 2),
               __builtin_amdgcn_alignbyte(lo[3], lo[2], 2), __builtin_amdgcn_alignbyte(hi[0], lo[3], 2)};
}

// Unsigned 6-bit weights (0..63) of the lane's four sets t from its ql chunks
// a (l), b (l + 32) and qh chunk h (quant.rs:155-159).
__device__ __forceinline__ void q6_sets(const u32x4& a, const u32x4& b, const u32x4& h,
                                        i32x4 (&q)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    q[0][k] = (int)((a[k] & 0x0f0f0f0fu) | ((h[k] << 4) & 0x30303030u));
    q[1][k] = (int)((b[k] & 0x0f0f0f0fu) | ((h[k] << 2) & 0x30303030u));
    q[2][k] = (int)(((a[k] >> 4) & 0x0f0f0f0fu) | (h[k] & 0x30303030u));
    q[3][k] = (int)(((b[k] >> 4) & 0x0f0f0f0fu) | ((h[k] >> 2) & 0x30303030u));
  }
}

// Fast-path dot of one block for one lane.
__device__ __forceinline__ float block_terms(const i32x4 (&q)[4], const int (&sc)[4], float d,
                                             const i32x4& a0, const i32x4& a1, const i32x4& a2,
                                             const i32x4& a3, int eb) {
  const i32x4 zero = {0, 0, 0, 0};
  const int m32 = (int)0xe0e0e0e0u;  // -32 in every byte
  const i32x4 neg32 = {m32, m32, m32, m32};
  i32x4 c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, q[0], zero, 0, 0, 0);
  i32x4 c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, q[1], zero, 0, 0, 0);
  i32x4 c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, q[2], zero, 0, 0, 0);
  i32x4 c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a3, q[3], zero, 0, 0, 0);
  c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, neg32, c0, 0, 0, 0);
  c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, neg32, c1, 0, 0, 0);
  c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, neg32, c2, 0, 0, 0);
  c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a3, neg32, c3, 0, 0, 0);
  int t[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    t[k] = mad_i24(sc[3], c3[k],
                   mad_i24(sc[2], c2[k], mad_i24(sc[1], c1[k], __mul24(sc[0], c0[k]))));
  const float tc =
      fmaf(fmaf(fmaf((float)t[3], 256.0f, (float)t[2]), 256.0f, (float)t[1]), 256.0f, (float)t[0]);
  return __builtin_amdgcn_ldexpf(d * tc, eb);
}

// Exact per-weight path of one block: xs = x of the block + 128 h + 16 s.
__device__ __forceinline__ float block_exact(const i32x4 (&q)[4], const int (&sc)[4], float d,
                                             const float* __restrict__ xs) {
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int qv = (int)(((uint32_t)q[t][i >> 2] >> (8 * (i & 3))) & 0xffu) - 32;
      acc = fmaf(k6_value_exact(d, sc[t], qv), xs[32 * t + i], acc);
    }
  }
  return acc;
}

// The same sum in the same order, one weight per iteration: for kernels that
// keep several vectors' state live, where the unrolled form's 64 loads in
// flight would crowd the registers.
__device__ __forceinline__ float block_exact_lean(const i32x4 (&q)[4], const int (&sc)[4],
                                                  float d, const float* __restrict__ xs) {
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
#pragma unroll 1
    for (uint32_t i = 0; i < 16u; ++i) {
      const uint32_t k = i >> 2;
      const uint32_t word = (uint32_t)(k == 0u   ? q[t][0]
                                       : k == 1u ? q[t][1]
                                       : k == 2u ? q[t][2]
                                                 : q[t][3]);
      const int qv = (int)((word >> (8u * (i & 3u))) & 0xffu) - 32;
      acc = fmaf(k6_value_exact(d, sc[t], qv), xs[32 * t + (int)i], acc);
    }
  }
  return acc;
}

// Largest |w| of the lane's share of a block: |d| * 32 * max |scale|.
__device__ __forceinline__ float q6_bound(const int (&sc)[4], float d) {
  const int m = max(max(abs(sc[0]), abs(sc[1])), max(abs(sc[2]), abs(sc[3])));
  return fabsf(d) * (float)(32 * m);
}

// NTOK activation vectors (batch-major x and y) share each decoded stage:
// vector t's images sit at img + t img_stride, and a launch with NTOK > 1
// gives every workgroup whole tiles (no split).  GROUPED: the rows are those
// of the group's matrices of one K, one after the other (every matrix but the
// last a whole number of tiles); tile t reads the matrix whose tiles reach
// past t.
//
// ARGMAX (one vector, one matrix): the greedy argmax of y under tie rule
// aa.rule, fused: each workgroup keeps the best candidate of the rows it
// stores, and the workgroups reduce theirs through the workspace's argmax
// area into *aa.result (argmax_device.h).
//
// SLICED (one vector, one matrix): a K-sliced launch (SliceArgs,
// mfma_common.h); the LDS holds the images and metadata of the workgroup's
// slice only, stage r of the matrix at local stage r - r_lo.
//
// PAIRED (one vector, one matrix of an odd block count nr): the launch sees
// rows / 2 rows of nb = 2 nr blocks, row r being rows 2 r and 2 r + 1 of the
// matrix one after the other.  Such a pair of rows starts on a 4-byte
// boundary (the rows themselves alternate by 2 bytes), so the two-block
// stages and their copies are the even case's.  Block b of a launch row
// meets x block b mod nr (x sits twice in the image area); the sums of its
// blocks b < nr go to y[2 r] and the rest to y[2 r + 1], the stage that
// holds blocks nr - 1 and nr handing one sum to each.
struct ArgmaxArgs {
  uint64_t* result;
  uint32_t rule;
};
template <int WAVES, int DEPTH, int NTOK, bool GROUPED, bool ARGMAX = false, bool SLICED = false,
          bool PAIRED = false>
__global__ __launch_bounds__(WAVES * 64) void q6k_matvec_mfma(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, uint32_t rows,
                                                              uint32_t nb, void* __restrict__ wsp,
                                                              SchedArgs sa, uint32_t prefetch,
                                                              GroupArgs ga, ArgmaxArgs aa,
                                                              SliceArgs sla) {
  static_assert(!ARGMAX || (NTOK == 1 && !GROUPED), "argmax over one matrix and vector");
  static_assert(!SLICED || (NTOK == 1 && !GROUPED && !ARGMAX), "slices of one matrix and vector");
  static_assert(!PAIRED || (NTOK == 1 && !GROUPED), "row pairs of one matrix");
  static_assert(!(PAIRED && SLICED && ARGMAX), "sliced row pairs: no argmax");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  if constexpr (GROUPED) load_group_args_early(ga);
  const uint32_t slots = sa.packed & 0xffu;
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + 1u) / 2u;
  // the schedule: whole and split tiles (sc), or K slices (ss)
  Sched sc{};
  SliceSched ss{};
  if constexpr (SLICED)
    ss = make_slice_sched(ntiles, sla, sa);
  else
    sc = make_sched(ntiles, nstages, WAVES, sa);
  // the stages whose images the LDS holds: [st0, st0 + nst), local index st - st0
  const uint32_t st0 = SLICED ? ss.r_lo : 0u;
  const uint32_t nbl = SLICED ? 2u * ss.ns : nb;
  const Layout L = layout(WAVES, DEPTH, SLICED ? 2u * ss.pstride : nb, slots, NTOK, PAIRED ? 2u : 1u);
  const uint32_t nr = nb / 2u;  // PAIRED: blocks of one matrix row
  const SplitWs ws = split_ws(wsp);
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t half = grp >> 1, sub = grp & 1u;
  const uint32_t row_bytes = nb * kQ6Bytes;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  uint8_t* const wstage = smem + wave * DEPTH * kStageBytes;

  // 1. x into the image area, natural order (block b of vector t at
  //    img + t img_stride + 1024 b)
  if constexpr (PAIRED) {
    // x twice over; a slice, the stretch of it that its stages meet
    copy_x<WAVES>(smem, L.img, x, nbl, wave, lane, nr, 2u * st0);
  } else {
#pragma unroll
    for (int t = 0; t < NTOK; ++t)
      copy_x<WAVES>(smem, L.img + t * L.img_stride,
                    x + (size_t)t * nb * kBlockElems + (size_t)2u * st0 * kBlockElems, nbl, wave,
                    lane);
  }

  // 2. this wave's pairs k = wave, wave + WAVES, ... of the workgroup's pairs
  //    (pair_at: a tile and its stage) and the copies of its first DEPTH, pair
  //    j into buffer j % DEPTH.  Copy i, lane l moves
  //    piece 4 i + l / 16 of row l % 16; the 16 lanes whose piece would be the
  //    28th re-read the 27th (same addresses, no extra traffic).  All copies
  //    lie inside the stage's 420 bytes of their row.
  auto pair_of = [&](uint32_t k) -> Pair {
    if constexpr (SLICED)
      return pair_at(ss, k);
    else
      return pair_at(sc, k, nstages);
  };
  const uint32_t npairs = SLICED ? ss.npairs : sc.npairs;
  const uint32_t voff = n * row_bytes + 16u * grp;
  const uint32_t voff_last = n * row_bytes + (grp < 2u ? 16u * (24u + grp) : kLastPiece);
  const uint32_t my_pairs = wave < npairs ? (npairs - 1u - wave) / WAVES + 1u : 0u;
  // the stage bytes of a pair's tile and the tile's row count
  auto tile_at = [&](const Pair& pr, uint32_t& nrows) -> const uint8_t* {
    uint32_t row0 = pr.tile * 16u, mrows = rows;
    const uint8_t* wm = w;
    if constexpr (GROUPED) {
      wm = ga.w[0];
      mrows = ga.rows[0];
#pragma unroll
      for (uint32_t k = 1; k < kMaxGroup; ++k)
        if (pr.tile >= ga.tile_end[k - 1]) {
          wm = ga.w[k];
          mrows = ga.rows[k];
          row0 = (pr.tile - ga.tile_end[k - 1]) * 16u;
        }
    }
    nrows = min(16u, mrows - row0);
    return wm + (size_t)row0 * row_bytes + kStageRowBytes * pr.r;
  };
  auto issue = [&](uint32_t j) {
    const Pair pr = pair_of(wave + j * WAVES);
    const uint32_t st = pr.r;
    uint32_t nrows;
    const uint8_t* sb = tile_at(pr, nrows);
    // the descriptor ends at the tile's last row: pieces past it read zero
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - kStageRowBytes * st),
        kBufferWord3);
    uint8_t* dst = wstage + (j % DEPTH) * kStageBytes;
#pragma unroll
    for (int i = 0; i < (int)kCopies - 1; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst + 1024 * i), 16,
                                                voff + 64u * i, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst + 1024 * (kCopies - 1)), 16,
                                              voff_last, 0, 0, 0);
  };
  // A long image build (48 blocks or more in the workgroup's range, every
  // wave a builder): the ring slots are set and a barrier passed first, so
  // that every wave's x copies go out ahead of all weight copies, and a
  // builder past the first round of waves (one per SIMD) builds before it
  // issues its own copies -- the memory queue, full of the first round's
  // copies, would hold it at them, and its images, for microseconds (the
  // 68-block down projection's images were done 3 us later that way).
  const bool long_build = nbl >= 48u;
  if (long_build) {
    init_slots<WAVES>(sbase, L, slots);
    lds_wait();
    __builtin_amdgcn_s_barrier();
  }
  const bool build_first = long_build && wave >= 4u && 4u * wave < nbl;
  // With one stage in flight, up to `prefetch` (<= 2) later pairs of the wave
  // are touched into L2 while the images are built: every 128-byte line of
  // their rows' 420 bytes is read 4 bytes wide (offsets 0, 128, 256, 384 and
  // 416 of each row) into a 256-byte LDS sink past the layout that nothing
  // reads.  Their copies then find the lines in L2.
  const uint32_t npf = DEPTH == 1 && my_pairs > 1u ? min(min(prefetch, 2u), my_pairs - 1u) : 0u;
  auto issue_first = [&]() {
#pragma unroll
    for (int j = 0; j < DEPTH; ++j)
      if ((uint32_t)j < my_pairs) issue(j);
    for (uint32_t j = 1; j <= npf; ++j) {
      const Pair pr = pair_of(wave + j * WAVES);
      uint32_t nrows;
      const uint8_t* sb = tile_at(pr, nrows);
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - kStageRowBytes * pr.r),
          kBufferWord3);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(smem + L.total), 4,
                                                n * row_bytes + 128u * grp, 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(smem + L.total), 4,
                                                n * row_bytes + kStageRowBytes - 4u, 0, 0, 0);
    }
  };
  if (!build_first) issue_first();

  // 3. ring slots (unless set above), then (once the x copies have landed)
  //    digit images and exponents
  if (!long_build) init_slots<WAVES>(sbase, L, slots);
  // the stage copies (then the touches) were issued after x's and complete in
  // order
  const uint32_t early = build_first ? 0u : min((uint32_t)DEPTH, my_pairs);
  if (early >= 3u)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * kCopies));
  else if (early == 2u)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kCopies));
  else if (early == 1u && npf == 2u)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies + 4));
  else if (early == 1u && npf == 1u)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies + 2));
  else if (early == 1u)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
  else
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  // chunk c = 8 h + 2 t + s: MFMA t of lane group 2 h + s
#pragma unroll
  for (int t = 0; t < NTOK; ++t)
    build_images<WAVES>(sbase, L, nbl, wave, grp, n, [](uint32_t c) {
      return 256u * ((c >> 1) & 3u) + 64u * (2u * (c >> 3) + (c & 1u));
    }, t);
  if (build_first) issue_first();
  lds_wait();
  __builtin_amdgcn_s_barrier();

  // 4. the wave's pairs
  const bool upper = half != 0u;  // lane groups 2, 3: scales 8..15
  const uint32_t base = sbase + wave * DEPTH * kStageBytes + 16u * n;
  const uint32_t qa0 = base + 256u * (4u * half + sub);
  const uint32_t qh0 = base + 256u * (8u + 2u * half + sub);
  const uint32_t sc0 = base + 256u * 12u;
  const uint32_t sb_lo = 8u * sub, sb_hi = 8u * sub + 16u;  // bit offsets of the lane's scales
  i32x4 A[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) A[t] = i32x4{0, 0, 0, 0};
  uint64_t best = 0u;  // ARGMAX: the best candidate of the rows this lane stored
  uint32_t fail = 0u;  // a bounded wait that gave up (kDevErr*)
  for (uint32_t j = 0; j < my_pairs; ++j) {
    const Pair pr = pair_of(wave + j * WAVES);
    const uint32_t st = pr.r, ls = st - st0;  // matrix stage, LDS stage
    const uint32_t later = min((uint32_t)DEPTH - 1u, my_pairs - 1u - j);
    if (DEPTH >= 3 && later >= 2u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kCopies));
    else if (DEPTH >= 2 && later >= 1u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const uint32_t buf = (j % DEPTH) * kStageBytes;
    u32x4 v[13];
    lds_read_stage(qa0 + buf, qh0 + buf, sc0 + buf, v);
    if (j + DEPTH < my_pairs) issue(j + DEPTH);  // the buffer just read is free again
    lds_read_images(sbase + L.img + 2048u * ls + 16u * n, kActiveLanes, A);
    u32x2 ex;
    uint32_t cnt;
    lds_read_expo(sbase + L.expo + 8u * ls, ex, cnt);
    const int e0 = __builtin_amdgcn_readfirstlane(ex[0]);
    const int e1 = __builtin_amdgcn_readfirstlane(ex[1]);

    // block 0: scales[8h + s + 2t] = bytes s, s + 2 of words 2h, 2h + 1 of v3
    i32x4 q0[4];
    q6_sets(v[0], v[1], v[2], q0);
    const uint32_t w0 = upper ? v[3][2] : v[3][0], w1 = upper ? v[3][3] : v[3][1];
    const int sc_0[4] = {scale_at(w0, sb_lo), scale_at(w0, sb_hi), scale_at(w1, sb_lo),
                         scale_at(w1, sb_hi)};
    const float d0 = half_bits_to_float(v[4][0] & 0xffffu);
    // block 1: its scale j < 14 is byte 2 + j of piece 25; scales 14, 15 and
    // d are the last word of piece 26
    i32x4 q1[4];
    q6_sets(skip2(v[5], v[6]), skip2(v[7], v[8]), skip2(v[9], v[10]), q1);
    const uint32_t u0 = upper ? v[11][2] : v[11][0], u1 = upper ? v[11][3] : v[11][1];
    const uint32_t u2 = upper ? v[12][3] : v[11][2];
    const int sc_1[4] = {scale_at(u0, sb_hi), scale_at(u1, sb_lo), scale_at(u1, sb_hi),
                         scale_at(u2, sb_lo)};
    const float d1 = half_bits_to_float(v[12][3] >> 16);

    if constexpr (NTOK > 1) {
      // the decoded stage meets every vector in turn (vector 0's images and
      // exponents are already in A, e0, e1); each vector's row sums go
      // straight to the tile's slot
      const uint32_t part_at = token_slot(sbase, L, sc.by_slots, pr, nstages, NTOK, lane, fail);
#pragma unroll 1
      for (uint32_t t = 0; t < (uint32_t)NTOK; ++t) {
        int f0 = e0, f1 = e1;
        uint32_t ct = cnt;
        if (t > 0u) {
          lds_read_images(sbase + L.img + t * L.img_stride + 2048u * st + 16u * n, kActiveLanes,
                          A);
          u32x2 et;
          lds_read_expo(sbase + L.expo + t * L.expo_stride + 8u * st, et, ct);
          f0 = __builtin_amdgcn_readfirstlane(et[0]);
          f1 = __builtin_amdgcn_readfirstlane(et[1]);
        }
        const float a0 = block_terms(q0, sc_0, d0, A[0], A[1], A[2], A[3], f0);
        const float a1 = block_terms(q1, sc_1, d1, A[4], A[5], A[6], A[7], f1);
        float pp[2] = {f0 != kBadBlock ? a0 : 0.0f, f1 != kBadBlock ? a1 : 0.0f};
        const float* const xs =
            x + (size_t)t * nb * kBlockElems + 512u * st + 128u * half + 16u * sub;
        const uint32_t counts = __builtin_amdgcn_readfirstlane(ct);
        uint32_t redo = 0u;
        if (counts != 0u) {
          const uint32_t list =
              sbase + L.expo + t * L.expo_stride + L.side_off + 2u * kSideBytes * st;
          redo = rounded_redo<2>(list, counts, grp, pp, [&](auto b) {
            return decltype(b)::value == 0 ? q6_bound(sc_0, d0) : q6_bound(sc_1, d1);
          });
        }
        if (f0 == kBadBlock || (redo & 1u)) pp[0] = block_exact_lean(q0, sc_0, d0, xs);
        if (f1 == kBadBlock || (redo & 2u)) pp[1] = block_exact_lean(q1, sc_1, d1, xs + 256);
        const float rowsum = sum_lane_groups(pp[0] + pp[1]);
        if (grp == 0u) lds_write_b32(part_at + 64u * t, __float_as_uint(rowsum));
      }
      token_slot_done<NTOK>(sbase, L, sc.by_slots, pr, nstages, lane, rows, y);
      continue;
    }

    const float c0 = block_terms(q0, sc_0, d0, A[0], A[1], A[2], A[3], e0);
    const float c1 = block_terms(q1, sc_1, d1, A[4], A[5], A[6], A[7], e1);
    float pp[2] = {e0 != kBadBlock ? c0 : 0.0f, e1 != kBadBlock ? c1 : 0.0f};
    const float* const xs = x + 512u * st + 128u * half + 16u * sub;
    const uint32_t counts = __builtin_amdgcn_readfirstlane(cnt);
    uint32_t redo = 0u;
    if (counts != 0u) {
      const uint32_t list = sbase + L.expo + L.side_off + 2u * kSideBytes * ls;
      redo = rounded_redo<2>(list, counts, grp, pp, [&](auto b) {
        return decltype(b)::value == 0 ? q6_bound(sc_0, d0) : q6_bound(sc_1, d1);
      });
    }
    if constexpr (PAIRED) {
      // the blocks' own x blocks (b mod nr) on the exact path, and each
      // block's sum to its row of the pair
      const uint32_t vb0 = 2u * st, vb1 = vb0 + 1u;
      const float* const x0 = x + 256u * (vb0 < nr ? vb0 : vb0 - nr) + 128u * half + 16u * sub;
      const float* const x1 = x + 256u * (vb1 < nr ? vb1 : vb1 - nr) + 128u * half + 16u * sub;
      if (e0 == kBadBlock || (redo & 1u)) pp[0] = block_exact(q0, sc_0, d0, x0);
      if (e1 == kBadBlock || (redo & 2u)) pp[1] = block_exact(q1, sc_1, d1, x1);
      float ra = 0.0f, rb = 0.0f;
      if (vb1 < nr) {
        ra = sum_lane_groups(pp[0] + pp[1]);
      } else if (vb0 >= nr) {
        rb = sum_lane_groups(pp[0] + pp[1]);
      } else {
        ra = sum_lane_groups(pp[0]);
        rb = sum_lane_groups(pp[1]);
      }
      if constexpr (SLICED)
        hand_off_slice<true>(sbase, L, ss, pr, ra, lane, rows, y, ws, fail, rb);
      else
        hand_off<1, ARGMAX, true>(sbase, L, slots, sc, sa, pr, nstages, ra, lane, rows, y, ws,
                                  fail, &best, aa.rule, rb);
      continue;
    }
    if (e0 == kBadBlock || (redo & 1u)) pp[0] = block_exact(q0, sc_0, d0, xs);
    if (e1 == kBadBlock || (redo & 2u)) pp[1] = block_exact(q1, sc_1, d1, xs + 256);
    const float rowsum = sum_lane_groups(pp[0] + pp[1]);

    // hand the 16 row partials to the tile's slot; the last stage finishes it
    if constexpr (SLICED)
      hand_off_slice(sbase, L, ss, pr, rowsum, lane, rows, y, ws, fail);
    else
      hand_off<1, ARGMAX>(sbase, L, slots, sc, sa, pr, nstages, rowsum, lane, rows, y, ws, fail,
                          &best, aa.rule);
  }
  if (fail != 0u) report_device_error(wsp, fail);
  if constexpr (ARGMAX) {
    // the workgroup's best, once every wave is done with the LDS, then the
    // grid's through the workspace
    best = wave_max_u64(best);
    __syncthreads();
    uint64_t* const wave_best = reinterpret_cast<uint64_t*>(smem);
    if (lane == 0u) wave_best[wave] = best;
    __syncthreads();
    if (wave == 0u) {
      const uint64_t m = lane < (uint32_t)WAVES ? wave_best[lane] : 0u;
      argmax_publish_wave(wave_max_u64(m), wsp, aa.result, lane);
    }
  }
}

// ---- Several activation vectors in the MFMA rows ---------------------------
//
// A pass over the weights with up to sixteen activation vectors (matmul-many,
// replacing si_q6_k_matmul_many, metal.rs:1052-1262; the batched head of
// qwen35_runtime.rs:2194-2197 takes up to eight candidates) puts the vectors
// in the rows of the A operand of v_mfma_i32_16x16x32_i8, so that each
// decoded weight meets them in few instructions.  K = 32 is one 32-element
// chunk j of a block, which spans two of its scales (2 j, 2 j + 1):
//
//  * B lane (k, n) holds weights 8 k .. 8 k + 7 of chunk j for tile row n as
//    the int8 4 (q - 32): (q ^ 32) << 2 puts q - 32 in two's complement in
//    bits 2..7, so each weight takes one mask-and-merge of its ql nibble and
//    its qh pair (the pairs XORed with 0b10 once per slice of qh).
//  * A row 4 (2 v + h) + d holds digit d of vector 4 G + 2 q + v over the
//    chunk's elements 16 h .. 16 h + 15 (scale 2 j + h) and zero elsewhere,
//    from group G's images (tokens_common.h): lane (k, i) reads its 8 bytes
//    only when k / 2 is its row's h; the other lanes hold zeros for the whole
//    kernel.  Two MFMAs per chunk and group of four vectors (q in {0, 1}):
//    groups G < NG, NG = 1, 2 or 4.
//  * Result lane (2 v + h, n) holds the four digit sums of vector
//    4 G + 2 q + v, row n, over scale 2 j + h alone, so T_d += sc C_d in
//    integers (|C_d| <= 2^18, |T_d| < 2^29) and per block the lane adds
//    d (sum_d 256^d T_d) 2^(eb - 2), eb the block's stored exponent (x = X
//    2^eb) and 2^-2 the weights' factor 4.  The lanes h = 0 and 1 of a vector
//    and row hold its even and odd scales; they are added once per tile.
//
// K slices.  Each group's images take 4 KB per block, so a launch cuts K
// into S slices of nbs blocks: workgroup g works on slice g / GS for tiles
// g % GS, g % GS + GS, ..., keeping that slice's images; each wave takes
// whole (tile, slice) pairs, their two-block stages one after another (the
// next stage's copy in flight while it computes), and stores each vector's
// and row's sum over the slice in the scratch; tok_reduce adds the S sums
// in slice order.  Side elements of a block (up to kSideMax, listed by the
// image build) are added as w_i x_i with w_i decoded exactly from the stage
// buffer before the next copy overwrites it; a rounded block is checked as
// in the one-vector kernel.  A (vector, row) that meets a block on the exact
// path, or whose rounded-block check fails, stores kPartRedo for the slice,
// and tok_reduce recomputes that slice exactly.
constexpr uint64_t kTokActiveLanes = 0xF0F0F0F00F0F0F0Full;  // lane (k, i): k / 2 == (i / 4) % 2

struct Q6TokArgs {
  uint32_t slices, groups_per_slice, m_gps, nbs;
  uint32_t m_slices;  // XCD-grouped launches: the division constant of the slice count
  uint32_t xcd;       // 1: the slices of a tile group share an XCD (GS a multiple of 8)
  void* wsp;          // the workspace, for failure reports
};

// LDS map: per-wave stage buffers, then ng groups' images of nbl blocks and
// their metadata (4 ng vectors); one unused ring slot.
__host__ __device__ constexpr Layout tok6_layout(uint32_t waves, uint32_t nbl, uint32_t depth,
                                                 uint32_t ng) {
  return make_layout(kStageBytes, 2u, 32u, waves, depth, nbl, 1u, 1u, 4u * ng);
}

// The lane's share of a two-block stage buffer (piece p of row n at 256 p +
// 16 n; a0 = buffer + 16 n + 256 (k / 2) + 8 (k % 2), srow = buffer + 16 n):
// block 0's 8-byte ql slices (half h, t & 1) at a0 + 512 (2 h + (t & 1)), its
// qh slices h at a0 + 2048 + 512 h, its scales (piece 12) and the word that
// holds d (piece 13); block 1 starts 2 bytes into piece 13, so for each of
// its slices the 8 bytes that start 2 before it (from a0 + 3328) and the 4
// after those (from a2 = a0 + 3328 + 8, or + 248 where that crosses into the
// next piece), its scales 0..13 as bytes 2..15 of piece 25 and the word of
// scales 14, 15 and d (stage bytes 416..419: the last word of piece 26).
struct Stage6 {
  u32x2 ql0[4], qh0[2];
  u32x4 sc0;
  uint32_t dw0;
  u32x2 ql1[4], qh1[2];
  uint32_t ql1n[4], qh1n[2];
  u32x4 sc1;
  uint32_t tail1;
};
__device__ __forceinline__ void lds_read_stage6(uint32_t a0, uint32_t a2, uint32_t srow,
                                                Stage6& s) {
  asm volatile(
      "ds_read_b64 %0, %22\n"
      "ds_read_b64 %1, %22 offset:512\n"
      "ds_read_b64 %2, %22 offset:1024\n"
      "ds_read_b64 %3, %22 offset:1536\n"
      "ds_read_b64 %4, %22 offset:2048\n"
      "ds_read_b64 %5, %22 offset:2560\n"
      "ds_read_b128 %6, %24 offset:3072\n"
      "ds_read_b32 %7, %24 offset:3328\n"
      "ds_read_b64 %8, %22 offset:3328\n"
      "ds_read_b64 %9, %22 offset:3840\n"
      "ds_read_b64 %10, %22 offset:4352\n"
      "ds_read_b64 %11, %22 offset:4864\n"
      "ds_read_b64 %12, %22 offset:5376\n"
      "ds_read_b64 %13, %22 offset:5888\n"
      "ds_read_b32 %14, %23\n"
      "ds_read_b32 %15, %23 offset:512\n"
      "ds_read_b32 %16, %23 offset:1024\n"
      "ds_read_b32 %17, %23 offset:1536\n"
      "ds_read_b32 %18, %23 offset:2048\n"
      "ds_read_b32 %19, %23 offset:2560\n"
      "ds_read_b128 %20, %24 offset:6400\n"
      "ds_read_b32 %21, %24 offset:6668\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(s.ql0[0]), "=&v"(s.ql0[1]), "=&v"(s.ql0[2]), "=&v"(s.ql0[3]), "=&v"(s.qh0[0]),
        "=&v"(s.qh0[1]), "=&v"(s.sc0), "=&v"(s.dw0), "=&v"(s.ql1[0]), "=&v"(s.ql1[1]),
        "=&v"(s.ql1[2]), "=&v"(s.ql1[3]), "=&v"(s.qh1[0]), "=&v"(s.qh1[1]), "=&v"(s.ql1n[0]),
        "=&v"(s.ql1n[1]), "=&v"(s.ql1n[2]), "=&v"(s.ql1n[3]), "=&v"(s.qh1n[0]),
        "=&v"(s.qh1n[1]), "=&v"(s.sc1), "=&v"(s.tail1)
      : "v"(a0), "v"(a2), "v"(srow)
      : "memory");
}

// The A operands of chunks 2 JP and 2 JP + 1 of a block for (G, q) = (0, 0),
// (0, 1), (1, 0), (1, 1): group G's image of the block at i0 (G = 0) or i1,
// + 1024 JP + 128 q.  Only the lanes in kTokActiveLanes read; the others keep
// their zeros.
template <int JP>
__device__ __forceinline__ void lds_read_tok6_images(uint32_t i0, uint32_t i1, i32x4 (&a)[4]) {
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %[sv], exec\n"
      "s_mov_b64 exec, %[m]\n"
      "ds_read_b128 %0, %[p] offset:%[o0]\n"
      "ds_read_b128 %1, %[p] offset:%[o1]\n"
      "ds_read_b128 %2, %[r] offset:%[o0]\n"
      "ds_read_b128 %3, %[r] offset:%[o1]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "s_mov_b64 exec, %[sv]"
      : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), [sv] "=&s"(saved)
      : [p] "v"(i0), [r] "v"(i1), [m] "s"(kTokActiveLanes), [o0] "i"(1024 * JP),
        [o1] "i"(1024 * JP + 128)
      : "memory");
}

// The same for one group: (G, q) = (0, 0), (0, 1) into a[0], a[1].
template <int JP>
__device__ __forceinline__ void lds_read_tok6_images1(uint32_t i0, i32x4 (&a)[4]) {
  uint64_t saved;
  asm volatile(
      "s_mov_b64 %[sv], exec\n"
      "s_mov_b64 exec, %[m]\n"
      "ds_read_b128 %0, %[p] offset:%[o0]\n"
      "ds_read_b128 %1, %[p] offset:%[o1]\n"
      "s_waitcnt lgkmcnt(0)\n"
      "s_mov_b64 exec, %[sv]"
      : "+v"(a[0]), "+v"(a[1]), [sv] "=&s"(saved)
      : [p] "v"(i0), [m] "s"(kTokActiveLanes), [o0] "i"(1024 * JP), [o1] "i"(1024 * JP + 128)
      : "memory");
}

// Exponents of the stage's two blocks and their side counts (one byte each)
// for four of the lane's vectors, from their metadata at m[O .. O + 3]
// (already offset to the stage).
template <int O, int N>
__device__ __forceinline__ void lds_read_tok6_meta(const uint32_t (&m)[N], u32x2 (&ex)[N],
                                                   uint32_t (&cnt)[N]) {
  static_assert(O + 4 <= N || N == 2, "four vectors from O (or the two of one group)");
  if constexpr (N == 2) {
    asm volatile(
        "ds_read_b64 %0, %4\n"
        "ds_read_b64 %1, %5\n"
        "ds_read_u16 %2, %4 offset:512\n"
        "ds_read_u16 %3, %5 offset:512\n"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(ex[0]), "=&v"(ex[1]), "=&v"(cnt[0]), "=&v"(cnt[1])
        : "v"(m[0]), "v"(m[1])
        : "memory");
    return;
  }
  static_assert(kCountOff == 512, "the offset below");
  asm volatile(
      "ds_read_b64 %0, %8\n"
      "ds_read_b64 %1, %9\n"
      "ds_read_b64 %2, %10\n"
      "ds_read_b64 %3, %11\n"
      "ds_read_u16 %4, %8 offset:512\n"
      "ds_read_u16 %5, %9 offset:512\n"
      "ds_read_u16 %6, %10 offset:512\n"
      "ds_read_u16 %7, %11 offset:512\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(ex[O]), "=&v"(ex[O + 1]), "=&v"(ex[O + 2]), "=&v"(ex[O + 3]), "=&v"(cnt[O]),
        "=&v"(cnt[O + 1]), "=&v"(cnt[O + 2]), "=&v"(cnt[O + 3])
      : "v"(m[O]), "v"(m[O + 1]), "v"(m[O + 2]), "v"(m[O + 3])
      : "memory");
}

__device__ __forceinline__ uint32_t lds_read_u8(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_u8 %0, %1\ns_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(addr) : "memory");
  return v;
}

// Byte o (< 420) of row n of a stage buffer (srow = buffer + 16 n).
__device__ __forceinline__ uint32_t stage6_byte(uint32_t srow, uint32_t o) {
  return lds_read_u8(o < kLastPiece ? srow + 256u * (o >> 4) + (o & 15u)
                                    : srow + 256u * (kRowPieces - 1u) + (o - kLastPiece));
}

// quant.rs's value of element i of block b of the stage for row n (quant.rs:
// 145-171: half h = i / 128, t = (i / 32) % 4, l = i % 32), d the block's
// scale factor.
__device__ __forceinline__ float stage6_weight(uint32_t srow, uint32_t b, uint32_t i, float d) {
  const uint32_t ob = kQ6Bytes * b, h = i >> 7, t = (i >> 5) & 3u, l = i & 31u;
  const uint32_t lo = stage6_byte(srow, ob + 64u * h + 32u * (t & 1u) + l);
  const uint32_t hi = stage6_byte(srow, ob + 128u + 32u * h + l);
  const int sc = (int)(int8_t)stage6_byte(srow, ob + 192u + (i >> 4));
  const int q = (int)(((lo >> (4u * (t >> 1))) & 0xfu) | (((hi >> (2u * t)) & 3u) << 4)) - 32;
  return k6_value_exact(d, sc, q);
}

// The lane's 8 weights 4 (q - 32) of chunk 4 h + T from its ql slice (h, T & 1)
// and its qh slice h XORed with 0xAA in every byte.
template <int T>
__device__ __forceinline__ u32x2 q6_chunk(u32x2 ql, u32x2 qx) {
  u32x2 r;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const uint32_t lo = T >= 2 ? (ql[k] >> 2) & 0x3c3c3c3cu : (ql[k] << 2) & 0x3c3c3c3cu;
    const uint32_t hi = (T == 3 ? qx[k] : qx[k] << (6 - 2 * T)) & 0xc0c0c0c0u;
    r[k] = lo | hi;
  }
  return r;
}

// Largest |scale| among the four int8 bytes of w from byte `from`.
__device__ __forceinline__ int max_abs_i8(uint32_t w, int from = 0, int to = 4) {
  int m = 0;
  for (int k = from; k < to; ++k) m = max(m, abs(scale_at(w, 8u * k)));
  return m;
}

// Up to 4 NG vectors (vectors past ntok are zero and not stored): the slice
// partial sums part_out[(k * 4 NG + v) * rows + row] of slice k.  DEPTH
// stage buffers per wave: the copies of its next DEPTH pairs in flight.
// NG = 2 (eight vectors) or 4 (sixteen): GQ = 2 NG MFMAs per chunk, (G, q)
// = (gq / 2, gq % 2) for vectors 4 G + 2 q + v.
template <int WAVES, int DEPTH, int NG>
__global__ __launch_bounds__(WAVES * 64) void q6k_tokens_mfma(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              uint32_t rows, uint32_t nb,
                                                              uint32_t ntok,
                                                              float* __restrict__ part_out,
                                                              Q6TokArgs ta) {
  static_assert(NG == 1 || NG == 2 || NG == 4, "four, eight or sixteen vectors");
  constexpr int GQ = 2 * NG;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t vh = grp >> 1, hs = grp & 1u;  // result lanes: vector 4 G + 2 q + vh, scales 2 j + hs
  const uint32_t row_bytes = nb * kQ6Bytes;
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  uint8_t* const wstage = smem + wave * DEPTH * kStageBytes;

  // this workgroup's slice k (blocks blk0 .. blk0 + nbl - 1) and its tiles
  // tg, tg + GS, ...  Workgroups go to the eight XCDs round robin (workgroup
  // b to XCD b % 8); XCD-grouped, the S workgroups of a tile group are
  // b = 8 (S i + k) + x for tile group 8 i + x, so they share that XCD's L2,
  // where a row's line that two slices' runs share is then read once.
  const FastDiv by_gps{ta.groups_per_slice, ta.m_gps};
  uint32_t k, tg;
  if (ta.xcd != 0u) {
    const uint32_t i = blockIdx.x >> 3;
    const uint32_t q = quo(i, FastDiv{ta.slices, ta.m_slices});
    k = i - q * ta.slices;
    tg = 8u * q + (blockIdx.x & 7u);
  } else {
    k = quo(blockIdx.x, by_gps);
    tg = blockIdx.x - k * ta.groups_per_slice;
  }
  const uint32_t blk0 = k * ta.nbs, nbl = min(ta.nbs, nb - blk0);
  const uint32_t nst = nbl / 2u;
  const Layout L = tok6_layout(WAVES, nbl, DEPTH, NG);
  const uint32_t ntw = tg < ntiles ? quo(ntiles - 1u - tg, by_gps) + 1u : 0u;
  const uint32_t my_tiles = wave < ntw ? (ntw - 1u - wave) / WAVES + 1u : 0u;
  const uint32_t my_pairs = my_tiles * nst;

  // 1. the vectors' blocks of the slice into the image area
  copy_x_group<WAVES>(smem, L.img, x, nb, blk0, nbl, NG, ntok, wave, lane);

  // 2. the copy of a pair's stage into buffer buf: local tile lt (tile
  //    tg + lt GS), stage s of the slice.  Copy i, lane l moves piece
  //    4 i + l / 16 of row l % 16 (the 16 lanes of the 28th piece re-read the
  //    27th), all inside the stage's 420 bytes of their row; rows past the
  //    matrix read zero.  The wave's pairs go tile by tile, a tile's stages in
  //    order: (lti, sli) is the next pair to issue.
  const uint32_t voff = n * row_bytes + 16u * grp;
  const uint32_t voff_last = n * row_bytes + (grp < 2u ? 16u * (24u + grp) : kLastPiece);
  uint32_t lti = wave, sli = 0u;
  auto issue = [&](uint32_t buf) {
    const uint32_t lt = lti, s = sli;
    uint8_t* const dst = wstage + buf * kStageBytes;
    sli = sli + 1u == nst ? 0u : sli + 1u;
    lti = sli == 0u ? lti + WAVES : lti;
    const uint32_t row0 = (tg + lt * ta.groups_per_slice) * 16u;
    const uint32_t nrows = min(16u, rows - row0);
    const uint32_t st = blk0 / 2u + s;
    const uint8_t* sb = w + (size_t)row0 * row_bytes + kStageRowBytes * st;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - kStageRowBytes * st),
        kBufferWord3);
#pragma unroll
    for (int i = 0; i < (int)kCopies - 1; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst + 1024 * i), 16,
                                                voff + 64u * i, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst + 1024 * (kCopies - 1)), 16,
                                              voff_last, 0, 0, 0);
  };
  const uint32_t early = min((uint32_t)DEPTH, my_pairs);  // the copies issued first
  auto issue_first = [&]() {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d)
      if ((uint32_t)d < early) issue((uint32_t)d);
  };

  // 3. ring state (the builders' count), then the first copies and the group
  //    images (as in q4k_tokens_mfma: the first round of waves issues before
  //    the barrier, the rest after; a builder converts exactly the blocks it
  //    copied)
  const bool first_round = wave < 4u;
  if (first_round) issue_first();
  init_slots<WAVES>(sbase, L, 1u);
  lds_wait();
  __builtin_amdgcn_s_barrier();
  if (!first_round) issue_first();
  const uint32_t builders = min((uint32_t)WAVES, (uint32_t)NG * nbl);
  if (wave < builders) {
    // (the stage copies went out after the x copies and complete in order)
    if (DEPTH >= 2 && early >= 2u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kCopies));
    else if (early >= 1u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    build_group_images<WAVES>(sbase, L, nbl, NG, wave, lane);
    lds_wait();
    if (lane == 0u) (void)lds_add_rtn(sbase + L.ready, 1u);
  }

  // 4. the wave's pairs
  const uint32_t srow0 = sbase + wave * DEPTH * kStageBytes + 16u * n;
  const uint32_t a00 = srow0 + 256u * (grp >> 1) + 8u * (grp & 1u);
  const uint32_t a20 = a00 + 3328u + ((grp & 1u) ? 248u : 8u);
  // the A lane (k, i) = (grp, n): digit n % 4 of vector 2 q + n / 8 of a group
  const uint32_t ibase = sbase + L.img + 256u * grp + 64u * (n >> 3) + 16u * (n & 3u);
  const uint32_t gstride = 4096u * nbl;
  // the metadata of the result lane's vectors 4 G + 2 q + vh, (G, q) = gq
  uint32_t meta[GQ];
#pragma unroll
  for (int gq = 0; gq < GQ; ++gq) meta[gq] = sbase + L.expo + (2u * gq + vh) * L.expo_stride;
  const uint32_t o_lo = 8u * hs, o_hi = 16u + 8u * hs;  // bit offsets of the lane's scales
  // per pair of groups: (G, q) = (2 p, 0), (2 p, 1), (2 p + 1, 0), (2 p + 1, 1)
  i32x4 A[(NG + 1) / 2][4];
#pragma unroll
  for (int pg = 0; pg < (NG + 1) / 2; ++pg)
#pragma unroll
    for (int i = 0; i < 4; ++i) A[pg][i] = i32x4{0, 0, 0, 0};
  float part[GQ];
#pragma unroll
  for (int gq = 0; gq < GQ; ++gq) part[gq] = 0.0f;
  uint32_t redo = 0u;  // bit gq: the slice of vector gq is recomputed exactly
  uint32_t lt = wave, sl = 0u;
  uint32_t fail = 0u;  // a bounded wait that gave up (kDevErr*)
  for (uint32_t p = 0; p < my_pairs; ++p) {
    // pair p's stage in buffer p % DEPTH, the copies of later pairs still out
    const uint32_t buf = DEPTH == 1 ? 0u : p % (uint32_t)DEPTH;
    if (DEPTH >= 2 && p + 1u < my_pairs)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCopies));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const uint32_t srow = srow0 + buf * kStageBytes;
    Stage6 sv;
    lds_read_stage6(a00 + buf * kStageBytes, a20 + buf * kStageBytes, srow, sv);
    if (p == 0u) wait_images(sbase, L, builders, fail);
    uint32_t m[GQ];
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) m[gq] = meta[gq] + 8u * sl;
    u32x2 ex[GQ];
    uint32_t cnt[GQ];
    lds_read_tok6_meta<0>(m, ex, cnt);
    if constexpr (GQ == 8) lds_read_tok6_meta<4>(m, ex, cnt);
    const float d0 = half_bits_to_float(sv.dw0 & 0xffffu);
    const float d1 = half_bits_to_float(sv.tail1 >> 16);

    // listed side elements, from the stage buffer before the next copy: the
    // h = 0 lane of each vector and row adds them
    uint32_t rounded = 0u;  // bit 2 gq + b: block b of vector gq is rounded
    uint32_t any_side = 0u;
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) any_side |= cnt[gq];
    if (__builtin_amdgcn_ballot_w64(any_side != 0u) != 0u) {
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
          const uint32_t c = (cnt[gq] >> (8 * b)) & 0xffu;
          if (c == kSideRounded) {
            rounded |= 1u << (2 * gq + b);
          } else if (hs == 0u) {
            const uint32_t list = meta[gq] + L.side_off + kSideBytes * (2u * sl + b);
            for (uint32_t e = 0; e < c; ++e) {
              const u32x2 ent = lds_read_b64(list + kSideEntryBytes * e);
              const float wv = stage6_weight(srow, (uint32_t)b, ent[0], b == 0 ? d0 : d1);
              part[gq] = fmaf(wv, __uint_as_float(ent[1]), part[gq]);
            }
          }
        }
      }
    }

    // the copy of pair p + DEPTH into the buffer just read: the stage is in
    // registers
    const bool last_stage = sl + 1u == nst;
    if (p + DEPTH < my_pairs) issue(buf);

    // the two blocks: per chunk four MFMAs and the integer scale combine
    float absp[GQ];
#pragma unroll
    for (int gq = 0; gq < GQ; ++gq) absp[gq] = 0.0f;
    const uint32_t ib0 = ibase + 4096u * (2u * sl);
    static_for<2>([&](auto bc) {
      constexpr int b = decltype(bc)::value;
      const uint32_t i0 = ib0 + 4096u * b;
      u32x2 ql[4], qx[2];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if constexpr (b == 0) {
          ql[c] = sv.ql0[c];
        } else {
          ql[c] = u32x2{__builtin_amdgcn_alignbyte(sv.ql1[c][1], sv.ql1[c][0], 2),
                        __builtin_amdgcn_alignbyte(sv.ql1n[c], sv.ql1[c][1], 2)};
        }
      }
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x2 qh = b == 0 ? sv.qh0[c]
                                : u32x2{__builtin_amdgcn_alignbyte(sv.qh1[c][1], sv.qh1[c][0], 2),
                                        __builtin_amdgcn_alignbyte(sv.qh1n[c], sv.qh1[c][1], 2)};
        qx[c] = u32x2{qh[0] ^ 0xaaaaaaaau, qh[1] ^ 0xaaaaaaaau};
      }
      int t[GQ][4];
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq)
#pragma unroll
        for (int d = 0; d < 4; ++d) t[gq][d] = 0;
      // software-pipelined: chunk j's four MFMAs go out before chunk j - 1's
      // products are added, so that no MFMA result is read right after its
      // MFMA
      i32x4 cp[GQ];
      int scp = 0;
      static_for<9>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        i32x4 c[GQ];
        int sc = 0;
        if constexpr (j < 8) {
          constexpr int h = j >> 2, tt = j & 3;
          if constexpr ((j & 1) == 0 && NG == 1) {
            lds_read_tok6_images1<j / 2>(i0, A[0]);
          } else if constexpr ((j & 1) == 0) {
#pragma unroll
            for (int pg = 0; pg < NG / 2; ++pg)
              lds_read_tok6_images<j / 2>(i0 + 2u * pg * gstride, i0 + (2u * pg + 1u) * gstride,
                                          A[pg]);
          }
          const u32x2 wq = q6_chunk<tt>(ql[2 * h + (tt & 1)], qx[h]);
          // scale 2 j + hs: block 0 byte 2 j + hs of its 16; block 1 byte
          // 2 + 2 j + hs of piece 25 (j < 7) or byte hs of the tail word (j = 7)
          if constexpr (b == 0)
            sc = scale_at(sv.sc0[j >> 1], (j & 1) ? o_hi : o_lo);
          else if constexpr (j == 7)
            sc = scale_at(sv.tail1, o_lo);
          else
            sc = scale_at(sv.sc1[(j + 1) >> 1], (j & 1) ? o_lo : o_hi);
          const int64_t bw = as_i64(wq[0], wq[1]);
          const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
          for (int gq = 0; gq < GQ; ++gq) {
            const i32x4& a = A[gq / 4][gq % 4];
            c[gq] = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                as_i64(a[2 * (j & 1)], a[2 * (j & 1) + 1]), bw, zero, 0, 0, 0);
          }
        }
        if constexpr (j > 0) {
#pragma unroll
          for (int gq = 0; gq < GQ; ++gq)
#pragma unroll
            for (int d = 0; d < 4; ++d) t[gq][d] = mad_i24(scp, cp[gq][d], t[gq][d]);
        }
        if constexpr (j < 8) {
#pragma unroll
          for (int gq = 0; gq < GQ; ++gq) cp[gq] = c[gq];
          scp = sc;
        }
      });
      const float db = b == 0 ? d0 : d1;
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq) {
        const int eb = (int)ex[gq][b];
        const float tc = fmaf(fmaf(fmaf((float)t[gq][3], 256.0f, (float)t[gq][2]), 256.0f,
                                   (float)t[gq][1]),
                              256.0f, (float)t[gq][0]);
        const float v = __builtin_amdgcn_ldexpf(db * tc, eb - 2);
        const bool bad = eb == kBadBlock;
        part[gq] += bad ? 0.0f : v;
        absp[gq] += bad ? 0.0f : fabsf(v);
        redo |= (uint32_t)bad << gq;
      }
    });

    // rounded blocks: the bound of their rounding against kRoundedTol of the
    // stage's sum |partial| of the vector and row (both lanes h = 0, 1)
    if (__builtin_amdgcn_ballot_w64(rounded != 0u) != 0u) {
      const float bound0 =
          fabsf(d0) * (float)(32 * max(max(max_abs_i8(sv.sc0[0]), max_abs_i8(sv.sc0[1])),
                                        max(max_abs_i8(sv.sc0[2]), max_abs_i8(sv.sc0[3]))));
      const float bound1 =
          fabsf(d1) * (float)(32 * max(max(max_abs_i8(sv.sc1[0], 2), max_abs_i8(sv.sc1[1])),
                                        max(max(max_abs_i8(sv.sc1[2]), max_abs_i8(sv.sc1[3])),
                                            max_abs_i8(sv.tail1, 0, 2))));
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq) {
        auto a2s = __builtin_amdgcn_permlane16_swap(__float_as_uint(absp[gq]),
                                                    __float_as_uint(absp[gq]), false, false);
        const float a = __uint_as_float(a2s[0]) + __uint_as_float(a2s[1]);
        float err = 0.0f;
        const uint32_t list = meta[gq] + L.side_off + kSideBytes * (2u * sl);
        if ((rounded >> (2 * gq)) & 1u) err = fmaf(bound0, rounded_err_all(list), err);
        if ((rounded >> (2 * gq + 1)) & 1u)
          err = fmaf(bound1, rounded_err_all(list + kSideBytes), err);
        if (!(err * 1.01f <= kRoundedTol * (a - err))) redo |= 1u << gq;
      }
    }

    if (last_stage) {
      // the tile's sums over the slice: lanes h = 0, 1 added; lane h stores
      // (G, q) = gq for gq in [h NG, h NG + NG), vector 2 gq + vh
      float tot[GQ];
      uint32_t rd = 0u;
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq) {
        auto s2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(part[gq]),
                                                   __float_as_uint(part[gq]), false, false);
        tot[gq] = __uint_as_float(s2[0]) + __uint_as_float(s2[1]);
      }
      {
        auto r2 = __builtin_amdgcn_permlane16_swap(redo, redo, false, false);
        rd = r2[0] | r2[1];
      }
      const uint32_t row = (tg + lt * ta.groups_per_slice) * 16u + n;
      if (row < rows) {
        float* const out = part_out + (size_t)k * (4u * NG) * rows + row;
#pragma unroll
        for (int gq = 0; gq < GQ; ++gq) {
          const uint32_t v = 2u * gq + vh;
          if ((uint32_t)(gq / NG) == hs && v < ntok)
            out[(size_t)v * rows] = ((rd >> gq) & 1u) ? __uint_as_float(kPartRedo) : tot[gq];
        }
      }
#pragma unroll
      for (int gq = 0; gq < GQ; ++gq) part[gq] = 0.0f;
      redo = 0u;
    }
    sl = last_stage ? 0u : sl + 1u;
    lt = last_stage ? lt + WAVES : lt;
  }
  if (fail != 0u) report_device_error(ta.wsp, fail);
}

// P: rows and nb are the launch's (row pairs of a matrix of nb / 2 blocks).
template <int W, int D, int NT = 1, bool G = false, bool AM = false, bool P = false>
bool launch_wd(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
               const Workspace& ws, hipStream_t s, hipError_t* err,
               const GroupArgs& ga = GroupArgs{}, const ArgmaxArgs& aa = ArgmaxArgs{}) {
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + 1u) / 2u;
  // several vectors: whole tiles only
  const LaunchShape ls = launch_shape(ntiles, nstages, W, NT == 1 ? ws.bytes : 0u, P ? 2u : 1u);
  const uint32_t grid = ls.groups;
  const uint32_t slots = ring_slots(W, D, ls.tiles_per_group, P ? 2u * nstages : nstages);
  // One pair touched ahead pays where the image build is long (the 68-block
  // down projection: 1 us of 22); with 20 blocks (the output head) it costs.
  static const int pf_env = env_int("SI_HIP_Q6K_PREFETCH", -1);
  const uint32_t prefetch = pf_env >= 0 ? (uint32_t)pf_env : (nb >= 48u ? 1u : 0u);
  const uint32_t lds =
      layout(W, D, nb, slots, NT, P ? 2u : 1u).total + (D == 1 && prefetch ? 256u : 0u);
  SchedArgs sa;
  if (lds > kLdsBytes || !make_sched_args(ntiles, nstages, slots, ls, &sa)) return false;
  // the argmax: an entry per workgroup, the waves' candidates at the LDS start
  if (AM && (grid > kArgmaxMaxGroups || (P ? 2u : 1u) * (uint64_t)rows >= kArgmaxMaxRows ||
             ws.bytes < kWorkspaceBytes))
    return false;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&q6k_matvec_mfma<W, D, NT, G, AM, false, P>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q6k_matvec_mfma<W, D, NT, G, AM, false, P>), dim3(grid), dim3(W * 64), lds,
                     s, w, x, y, rows, nb, ws.ptr, sa, D == 1 ? prefetch : 0u, ga, aa,
                     SliceArgs{});
  *err = hipGetLastError();
  return true;
}

// A K-sliced launch in S slices (false when the shape or the LDS does not fit).
// P: row pairs, rows and nb being the pairs' (rows / 2 rows of 2 nr blocks).
template <int W, int D, bool P = false>
bool launch_sliced(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                   uint32_t S, const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = nb / 2u;
  // even nb (4-byte aligned rows and stages); in-tile offsets (16 rows) and
  // descriptor sizes are 32-bit; the slice's blocks bound the LDS metadata
  if (rows == 0u || nb == 0u || (nb & 1u) != 0u || (uint64_t)nb * kQ6Bytes * 16u > 0x7fffffffu)
    return false;
  SliceShape sh;
  if (!slice_shape(ntiles, nstages, S, (uint32_t)cu_count(), ws.bytes, &sh, P ? 128u : 64u))
    return false;
  if (2u * sh.ns_max > kMaxMetaBlocks) return false;
  const uint32_t slots = ring_slots(W, D, sh.tiles_per_group, sh.ns_max);
  static const int pf_env = env_int("SI_HIP_Q6K_PREFETCH", -1);
  const uint32_t prefetch = D == 1 && pf_env > 0 ? (uint32_t)pf_env : 0u;
  const uint32_t lds =
      layout(W, D, 2u * sh.ns_max, slots, 1u, P ? 2u : 1u).total + (prefetch ? 256u : 0u);
  if (lds > kLdsBytes || slots > 0xffu || sh.groups > 0xffffu) return false;
  SchedArgs sa{};
  sa.packed = (sh.groups << 16) | slots;
  sa.m_slots = div_magic(slots);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&q6k_matvec_mfma<W, D, 1, false, false, true, P>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q6k_matvec_mfma<W, D, 1, false, false, true, P>), dim3(sh.groups), dim3(W * 64),
                     lds, s, w, x, y, rows, nb, ws.ptr, sa, prefetch, GroupArgs{}, ArgmaxArgs{},
                     sh.args);
  *err = hipGetLastError();
  return true;
}

// Slices for a one-vector launch, or 0.  A workgroup builds the images of
// the blocks it reads before its first stage, about 0.07-0.1 us per block,
// and only its first stages (one per wave, plus a pair touched into L2) are
// in flight meanwhile; slicing shrinks the build S-fold but rounds each
// slice's stages and each workgroup's tiles up.  Measured (MI355X, us):
//   rows x cols      unsliced  S = 2   S = 4
//   640 x 17408        12.1     11.0     8.3
//   2560 x 17408       18.4     19.1    15.2
//   2048 x 16384       13.3     10.8    10.0
//   512 x 12288        10.9      8.3     7.3
//   4096 x 14336       16.2     17.0    16.3
//   5120 x 17408       24.5     27.2    25.7
//   8192 x 28672       57.0     52.4    56.0
//   2048 x 32768       50.4     20.2
//   2560 x 9728         9.5              9.7
// So: four slices when the unsliced launch's busiest workgroup has at most
// two rounds of pairs (24; its build is then exposed) and slicing adds it
// none or the rows are long (48 blocks or more); with more pairs, only when
// the unsliced images leave room for fewer than eight waves (very long
// rows), in the fewest slices that add no pairs to the busiest workgroup.
uint32_t q6_slices(uint32_t ntiles, uint32_t nb, size_t ws_bytes) {
  static const int env = env_int("SI_HIP_Q6K_SLICES", -1);
  if (env >= 0) return (uint32_t)env;
  const uint32_t nst = nb / 2u;
  if (nst < 16u) return 0u;
  const uint64_t cus = (uint64_t)cu_count();
  if (nb > kMaxMetaBlocks) {
    // rows longer than the unsliced kernel takes must slice: the fewest
    // slices (from four) whose images (64 blocks at most) leave the stage
    // buffers of 12 waves room in the LDS
    uint32_t S = 4u;
    while (S < 64u && S < cus && (nst + S - 1u) / S > 32u) S *= 2u;
    return S;
  }
  // the unsliced launch's busiest workgroup (launch_shape's choice at 12 waves)
  const LaunchShape ls = launch_shape(ntiles, nst, 12u, ws_bytes, 1u);
  const uint64_t g1 = ls.groups;
  const uint64_t q = ntiles / g1, lp = (ntiles - q * g1) * nst;
  const uint64_t most0 = ls.split ? q * nst + (lp + g1 - 1u) / g1 : (ntiles + g1 - 1u) / g1 * nst;
  auto most = [&](uint32_t S) {  // the busiest sliced workgroup's pairs
    const uint64_t gs = std::min<uint64_t>(ntiles, cus / S);
    return (ntiles + gs - 1u) / gs * ((nst + S - 1u) / S);
  };
  if (most0 <= 24u) return most(4u) <= most0 || nb >= 48u ? 4u : 0u;
  if (layout(8u, 1u, nb, 2u).total <= kLdsBytes) return 0u;
  for (uint32_t S : {2u, 4u})
    if (most(S) <= most0) return S;
  return 0u;
}

// An odd block count over an even row count runs as row pairs (PAIRED) of
// 2 nb blocks.
bool q6_shape_ok(uint32_t rows, uint32_t nb);
bool paired_ok(uint32_t rows, uint32_t nb) {
  return (nb & 1u) == 1u && rows >= 2u && (rows & 1u) == 0u && q6_shape_ok(rows / 2u, 2u * nb);
}

// even nb (4-byte aligned rows and stages); in-tile offsets (16 rows) and the
// descriptor sizes are 32-bit
bool q6_shape_ok(uint32_t rows, uint32_t nb) {
  return nb != 0 && (nb & 1u) == 0 && nb <= kMaxMetaBlocks && rows != 0 &&
         (uint64_t)nb * kQ6Bytes * 16u <= 0x7fffffffu &&
         (uint64_t)nb * 1024u <= 0x7fffffffu &&
         (uint64_t)((rows + 15u) / 16u) * (nb / 2u) <= 0xffffffffu &&
         quotients_fit((rows + 15u) / 16u, nb / 2u);
}

}  // namespace

namespace {
// An odd block count nb over an even row count: row pairs, K-sliced by the
// rule of the even case (and always past 64 blocks, where the pairs' rows
// exceed what the unsliced kernel takes), else unsliced.
bool launch_pairs(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                  bool may_slice, const Workspace& ws, hipStream_t s, hipError_t* err) {
  if ((nb & 1u) == 0u || rows < 2u || (rows & 1u) == 1u) return false;
  const uint32_t prows = rows / 2u, pnb = 2u * nb;
  if (may_slice) {
    const uint32_t S = q6_slices((prows + 15u) / 16u, pnb, ws.bytes);
    if (S >= 2u && (launch_sliced<12, 1, true>(w, x, y, prows, pnb, S, ws, s, err) ||
                    launch_sliced<8, 1, true>(w, x, y, prows, pnb, S, ws, s, err)))
      return true;
  }
  return paired_ok(rows, nb) &&
         (launch_wd<12, 1, 1, false, false, true>(w, x, y, prows, pnb, ws, s, err) ||
          launch_wd<10, 1, 1, false, false, true>(w, x, y, prows, pnb, ws, s, err) ||
          launch_wd<8, 1, 1, false, false, true>(w, x, y, prows, pnb, ws, s, err) ||
          launch_wd<4, 1, 1, false, false, true>(w, x, y, prows, pnb, ws, s, err));
}

// Up to eight vectors in one pass over the weights: q6k_tokens_mfma in K
// slices of nbs blocks, then tok_reduce.  false when the shape does not fit
// (q6_shape_ok, the slices' partial sums within the scratch, the LDS).
template <int W, int D, int NG>
bool launch_tok6(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                 uint32_t ntok, uint32_t nbs, const Workspace& ws, hipStream_t s,
                 hipError_t* err) {
  if (ntok == 0u || ntok > 4u * NG || nbs < 2u || (nbs & 1u) != 0u || !q6_shape_ok(rows, nb))
    return false;
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t cus = (uint32_t)cu_count();
  Q6TokArgs ta{};
  ta.nbs = min(nbs, nb);
  ta.slices = (nb + ta.nbs - 1u) / ta.nbs;
  if (ta.slices > cus || (size_t)ta.slices * 4u * NG * rows * sizeof(float) > ws.scratch_bytes)
    return false;
  ta.groups_per_slice = min(cus / ta.slices, ntiles);
  // XCD-grouped on request (SI_HIP_Q6K_TOK_XCD=1), when a multiple of 8 groups
  // per slice keeps nearly every CU busy (S = 2 on 256 CUs: all of them).  On
  // the head it cuts the L2 fills from 1.18 to 1.10 (four-block slices) or
  // 1.065 (ten-block slices) of the weight bytes but costs 4 us at M = 8, so
  // it is off by default.
  static const int xcd_env = env_int("SI_HIP_Q6K_TOK_XCD", 0);
  const uint32_t gs8 = ta.groups_per_slice & ~7u;
  if (xcd_env != 0 && ta.slices > 1u && gs8 >= 8u &&
      (uint64_t)gs8 * ta.slices * 16u >= (uint64_t)cus * 15u) {
    ta.groups_per_slice = gs8;
    ta.xcd = 1u;
    ta.m_slices = div_magic(ta.slices);
  }
  const uint32_t grid = ta.groups_per_slice * ta.slices;
  // block and tile indices divided by GS
  if ((uint64_t)(grid + ntiles) * ta.groups_per_slice >= (1ull << 32)) return false;
  ta.m_gps = div_magic(ta.groups_per_slice);
  ta.wsp = ws.ptr;
  const uint32_t lds = tok6_layout(W, ta.nbs, D, NG).total;
  if (lds > kLdsBytes) return false;
  static const hipError_t attr =
      hipFuncSetAttribute(reinterpret_cast<const void*>(&q6k_tokens_mfma<W, D, NG>),
                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q6k_tokens_mfma<W, D, NG>), dim3(grid), dim3(W * 64), lds, s, w, x, rows, nb, ntok,
                     ws.scratch, ta);
  *err = hipGetLastError();
  if (*err == hipSuccess) {
    launch_tok_reduce<kTypeQ6K>(ws.scratch, y, rows, ta.slices, 4u * NG, ntok, w, x, nb, ta.nbs, s);
    *err = hipGetLastError();
  }
  return true;
}

// The vectors-in-rows pass for ntok <= 16 vectors.  Up to eight: 12 waves
// with four-block slices, else (the partial sums of more slices than the
// scratch holds) the fewest slices whose images leave 8 waves their stage
// buffers.  Nine to sixteen: 8 waves with four-block slices, or false (the
// caller then runs passes of eight).
bool launch_tok6_any(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                     uint32_t ntok, const Workspace& ws, hipStream_t s, hipError_t* err) {
  static const int nbs_env = env_int("SI_HIP_Q6K_TOK_NBS", 0);
  static const int w_env = env_int("SI_HIP_Q6K_TOK_WAVES", 0);
  if (ntok <= 4u) {  // one group: 12 waves (16 on request)
    const uint32_t nbs = nbs_env > 0 ? (uint32_t)nbs_env : 4u;
    if (w_env == 16 ? launch_tok6<16, 1, 1>(w, x, y, rows, nb, ntok, nbs, ws, s, err)
                    : launch_tok6<12, 1, 1>(w, x, y, rows, nb, ntok, nbs, ws, s, err))
      return true;
  }
  if (ntok > 8u)  // sixteen vectors: 8 waves (the registers of four groups)
    return launch_tok6<8, 1, 4>(w, x, y, rows, nb, ntok, nbs_env > 0 ? (uint32_t)nbs_env : 4u,
                                ws, s, err);
  if (nbs_env > 0 || w_env > 0) {
    const uint32_t nbs = nbs_env > 0 ? (uint32_t)nbs_env : 4u;
    switch (w_env) {
      case 8: return launch_tok6<8, 1, 2>(w, x, y, rows, nb, ntok, nbs, ws, s, err);
      case 82: return launch_tok6<8, 2, 2>(w, x, y, rows, nb, ntok, nbs, ws, s, err);
      default: return launch_tok6<12, 1, 2>(w, x, y, rows, nb, ntok, nbs, ws, s, err);
    }
  }
  return launch_tok6<12, 1, 2>(w, x, y, rows, nb, ntok, 4u, ws, s, err) ||
         launch_tok6<12, 1, 2>(w, x, y, rows, nb, ntok, 6u, ws, s, err) ||
         launch_tok6<8, 1, 2>(w, x, y, rows, nb, ntok, 10u, ws, s, err);
}
}  // namespace

bool launch_q6k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  static const int cfg = env_int("SI_HIP_Q6K_MFMA_CFG", 0);
  if ((nb & 1u) == 1u && (rows & 1u) == 0u)
    return launch_pairs(w, x, y, rows, nb, cfg == 0, ws, s, err);
  if ((nb & 1u) == 1u && rows >= 3u && (uint64_t)rows * nb >= 65536u) {
    // an odd row count as well: the pairs of all rows but the last, then the
    // last row alone (one workgroup).  The second launch costs 3-5 us, so
    // below 64K blocks the generic kernel (one wave per row) is faster.
    if (!launch_pairs(w, x, y, rows - 1u, nb, cfg == 0, ws, s, err)) return false;
    if (*err == hipSuccess)
      *err = launch_row_dot(kTypeQ6K, w + (size_t)(rows - 1u) * nb * kQ6Bytes, x, y + (rows - 1u),
                            cols, s);
    return true;
  }
  if (cfg == 0 && nb > kMaxMetaBlocks) {  // (q6_shape_ok takes none of these)
    const uint32_t S = q6_slices((rows + 15u) / 16u, nb, ws.bytes);
    return S >= 2u && (launch_sliced<12, 1>(w, x, y, rows, nb, S, ws, s, err) ||
                       launch_sliced<8, 1>(w, x, y, rows, nb, S, ws, s, err));
  }
  if (!q6_shape_ok(rows, nb)) return false;
  switch (cfg) {
    case 1: return launch_wd<12, 1>(w, x, y, rows, nb, ws, s, err);
    case 2: return launch_wd<8, 2>(w, x, y, rows, nb, ws, s, err);
    case 3: return launch_wd<8, 1>(w, x, y, rows, nb, ws, s, err);
    case 4: return launch_wd<6, 2>(w, x, y, rows, nb, ws, s, err);
    default: break;
  }
  const uint32_t S = q6_slices((rows + 15u) / 16u, nb, ws.bytes);
  if (S >= 2u && (launch_sliced<12, 1>(w, x, y, rows, nb, S, ws, s, err) ||
                  launch_sliced<8, 1>(w, x, y, rows, nb, S, ws, s, err)))
    return true;
  return launch_wd<12, 1>(w, x, y, rows, nb, ws, s, err) || launch_wd<10, 1>(w, x, y, rows, nb, ws, s, err) ||
         launch_wd<8, 1>(w, x, y, rows, nb, ws, s, err) || launch_wd<4, 1>(w, x, y, rows, nb, ws, s, err);
}

bool launch_q6k_matvec_argmax_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                                   uint32_t cols, uint32_t rule, uint64_t* result,
                                   const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  const ArgmaxArgs aa{result, rule};
  if (paired_ok(rows, nb))
    return launch_wd<12, 1, 1, false, true, true>(w, x, y, rows / 2u, 2u * nb, ws, s, err,
                                                  GroupArgs{}, aa) ||
           launch_wd<8, 1, 1, false, true, true>(w, x, y, rows / 2u, 2u * nb, ws, s, err,
                                                 GroupArgs{}, aa);
  if (!q6_shape_ok(rows, nb)) return false;
  return launch_wd<12, 1, 1, false, true>(w, x, y, rows, nb, ws, s, err, GroupArgs{}, aa) ||
         launch_wd<8, 1, 1, false, true>(w, x, y, rows, nb, ws, s, err, GroupArgs{}, aa);
}

// batch >= 2 vectors: four, three or two per pass over the weights while
// their images fit the LDS beside the stage buffers (K up to about 5120 for
// four), one per pass otherwise.
bool launch_q6k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  if (!q6_shape_ok(rows, nb)) return false;
  static const int tok_min = env_int("SI_HIP_Q6K_TOKENS_MIN", 3);
  for (uint32_t b = 0; b < batch;) {
    const uint32_t left = batch - b;
    const float* xb = x + (size_t)b * cols;
    float* yb = y + (size_t)b * rows;
    uint32_t nt = 0;
    if (tok_min > 0 && left > 8u &&
        launch_tok6_any(w, xb, yb, rows, nb, min(16u, left), ws, s, err))
      nt = min(16u, left);
    else if (tok_min > 0 && left >= (uint32_t)tok_min &&
             launch_tok6_any(w, xb, yb, rows, nb, min(8u, left), ws, s, err))
      nt = min(8u, left);
    else if (left >= 4u && (launch_wd<8, 1, 4>(w, xb, yb, rows, nb, ws, s, err) ||
                       launch_wd<6, 1, 4>(w, xb, yb, rows, nb, ws, s, err)))
      nt = 4;
    else if (left == 3u && (launch_wd<8, 1, 3>(w, xb, yb, rows, nb, ws, s, err) ||
                            launch_wd<6, 1, 3>(w, xb, yb, rows, nb, ws, s, err)))
      nt = 3;
    else if (left >= 2u && (launch_wd<8, 1, 2>(w, xb, yb, rows, nb, ws, s, err) ||
                            launch_wd<6, 1, 2>(w, xb, yb, rows, nb, ws, s, err)))
      nt = 2;
    else if (launch_q6k_matvec_mfma(w, xb, yb, rows, cols, ws, s, err))
      nt = 1;
    if (nt == 0) {
      if (b == 0) return false;
      *err = hipErrorInvalidValue;
      return true;
    }
    if (*err != hipSuccess) return true;
    b += nt;
  }
  return true;
}

bool mfma::launch_q6k_matvec_group(const GroupArgs& ga, uint32_t total_rows, uint32_t cols,
                             const float* x, float* y, const Workspace& ws, hipStream_t s,
                             hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  if (!q6_shape_ok(total_rows, nb)) return false;
  return launch_wd<12, 1, 1, true>(ga.w[0], x, y, total_rows, nb, ws, s, err, ga) ||
         launch_wd<8, 1, 1, true>(ga.w[0], x, y, total_rows, nb, ws, s, err, ga);
}

}  // namespace sihip
