// Q4_K matvec on the gfx950 matrix cores (replaces si_q4_k_matvec* for one
// input vector, src/metal.rs:310-494).
//
// The dot of a 32-weight unit, sum_i q_i * x_i with q_i in 0..15, is done as
// an exact integer product on v_mfma_i32_16x16x64_i8:
//
//  * Activations.  Each 256-element block b of x is written in fixed point,
//    x_i = X_i * 2^(e_b - 30) with |X_i| <= 2^30 (e_b from the block's largest
//    |x|), and X_i = sum_d D_d * 256^d in four signed byte digits (|D| <= 128,
//    the top one <= 64).  Rounding x to X costs at most 2^-31 of the block's
//    largest activation.
//  * Weights.  A 16-byte piece of qs masked with 0x0f (or shifted by 4 first)
//    is 16 int8 weights.
//  * Units stay apart.  Lane l of the B operand is row l % 16 of a 16-row
//    tile; lane group g = l / 16 supplies the qs bytes [32g, 32g + 32) of the
//    block, i.e. units 2g (low nibbles) and 2g + 1 (high nibbles).  Rows
//    4g..4g+3 of the A operand hold the four digits of the activations that
//    meet group g's weights and are zero elsewhere, so output rows 4g + d are
//    digit d of group g's unit sums, and they land in lane group g -- the
//    lanes that hold that unit's scale and min.
//
// Per block and lane: C_e, C_o (4 digits each) from four MFMAs; T_d = sc_e *
// C_e[d] + sc_o * C_o[d] in integers (|T_d| < 2^23, exact in f32); y +=
// (d * (sum_d T_d * 256^d) - dmin * (m_e * X_e + m_o * X_o)) * 2^(e_b-30),
// X_u the sum of unit u's fixed-point activations (exact, rounded once), so
// both terms see the same rounded activations and, in exact arithmetic, the
// pair is sum_i w_i X_i 2^(e_b-30) with w_i the weight of quant.rs.  Their
// f32 rounding is bounded by 2^-21 (|d T| + |dmin| (m_e |X_e| + m_o |X_o|))
// per block, which can exceed the bar where w_i cancels inside its own decode
// (d sc q close to dmin m); every stage of a row checks that bound (stage_ok)
// and a row that fails recomputes the stage on the exact per-weight path, so
// the dot stays within 2e-5 * sum|w*x| on every input.  Blocks whose
// activations are not finite or reach 2^100 take the exact per-weight f32
// path instead, so NaN/Inf propagate as in the reference.
//
// Data path.  One persistent workgroup of WAVES waves per CU.  At start it
// turns all of x into digit images in LDS (1 KB per block, plus unit sums and
// exponents) while each wave's first stage of weights is already in flight.
// Workgroup g of G owns the 16-row tiles g, g + G, ...; their (tile,
// stage) pairs, a stage being four blocks (16 rows x 576 bytes), go to the
// waves round-robin, so every wave streams its own sequence of stages.
// Weights arrive by 16-byte buffer->LDS copies in piece-major order (LDS
// byte 16 (16 q + r) is piece q of row r), so every read is a conflict-free
// 16-lane sweep; a wave's next stage is in flight while it computes.  Only
// the 16 lanes whose A rows carry digits read images, two blocks at a time
// (exec-masked; the other lanes hold zeros for the whole kernel).  A wave leaves its stage's 16 row
// partials in an LDS slot of the tile and counts them with an LDS atomic; the
// wave that completes the tile sums the partials in stage order and stores
// the rows, so results do not depend on timing.  With MATS = 2 (fused SwiGLU
// gate/up, replacing si_q4_k_fused_gate_up, metal.rs:498-587) a tile's pairs
// cover the stages of both matrices, which share the activation images, and
// the finishing wave stores silu(gate) * up.  LDS is only touched through
// inline asm and the one barrier is a bare s_barrier: the compiler neither
// counts nor orders buffer->LDS copies, and a fence would drain them.
#include "mfma_common.h"
#include "si_hip_tuned.h"
#include "tokens_common.h"

namespace sihip {
namespace {

using namespace mfma;

// Block bytes of the two formats this kernel reads (QB = quant bits): 144
// (Q4_K) and 176 (Q5_K), both multiples of 16.  A stage is 16 rows x SB
// blocks (SB = 4, or 2 for the one-vector kernel's finer form): SB * 9 (or
// 11) 16-byte pieces per row, moved by stage_copies 64-lane copies, the last
// one's lanes past the row's pieces re-reading its last piece.
__host__ __device__ constexpr uint32_t block_bytes(int qb) { return qb == 5 ? kQ5Bytes : kQ4Bytes; }
__host__ __device__ constexpr uint32_t block_pieces(int qb) { return block_bytes(qb) / 16u; }
__host__ __device__ constexpr uint32_t stage_copies(int qb, int sb = 4) {
  return (16u * (uint32_t)sb * block_pieces(qb) + 63u) / 64u;
}
__host__ __device__ constexpr uint32_t stage_bytes(int qb, int sb = 4) {
  return 1024u * stage_copies(qb, sb);
}
static_assert(stage_bytes(4) == 64u * kQ4Bytes && stage_bytes(5) == 64u * kQ5Bytes,
              "four-block stages fill their copies exactly");

// Full-line copies (LINES: Q4_K in four-block stages, nb = 4 mod 8 blocks per
// row, the matrix 128-byte aligned).  A row's four blocks of a stage are 576
// bytes, four and a half 128-byte lines, and rows of 144 nb bytes start 64
// bytes apart modulo a line, so even rows start their even stages on a line
// and odd rows 64 bytes into one, the other way round in odd stages.  A stage
// moves as the five whole lines that hold it (the half line it shares with
// the next or the previous stage included): ten copies, copy (j, c) taking
// line j of the eight rows 2 i + c, lane 8 i + ((k + (i >> 1)) & 7) of it
// piece k of its row's line, into LDS region 2 j + (c ^ parity of the
// stage).  Every copy reads whole lines, which the nontemporal policy streams
// without fetching a line twice.  In odd stages lane n of the matrix-core
// layout takes row n ^ 1, so that every lane meets a row of one alignment in
// one LDS region at every stage and keeps one table of read addresses; a
// 16-lane read of one piece of the 16 rows meets 16 different LDS bank groups
// (the rotation by i >> 1 spreads the rows that share a line slot, and the
// two alignments sit half a line apart).
constexpr uint32_t kLineCopies = 10u;
constexpr uint32_t kLineStage = 1024u * kLineCopies;  // 16 rows x 5 lines
constexpr int kNontemporal = 2;                       // buffer cache policy: NT

// LDS map (make_layout): SB-block stages, 32 bytes of unit sums per block.
__host__ __device__ constexpr Layout layout(uint32_t waves, uint32_t depth, uint32_t nb,
                                            uint32_t slots, uint32_t mats, uint32_t ntok = 1u,
                                            int qb = 4, int sb = 4, bool lines = false) {
  return make_layout(lines ? kLineStage : stage_bytes(qb, sb), (uint32_t)sb, 32u, waves, depth,
                     nb, slots, mats, ntok);
}

// The lane's header and two qs pieces of the four blocks of a full-line stage
// buffer, each at its own address (a[3 b], a[3 b + 1], a[3 b + 2]) plus IMM.
template <int IMM>
__device__ __forceinline__ void lds_read_weights_at(const uint32_t (&a)[12], u32x4 (&v)[12]) {
  asm volatile(
      "ds_read_b128 %0, %12 offset:%24\n"
      "ds_read_b128 %1, %13 offset:%24\n"
      "ds_read_b128 %2, %14 offset:%24\n"
      "ds_read_b128 %3, %15 offset:%24\n"
      "ds_read_b128 %4, %16 offset:%24\n"
      "ds_read_b128 %5, %17 offset:%24\n"
      "ds_read_b128 %6, %18 offset:%24\n"
      "ds_read_b128 %7, %19 offset:%24\n"
      "ds_read_b128 %8, %20 offset:%24\n"
      "ds_read_b128 %9, %21 offset:%24\n"
      "ds_read_b128 %10, %22 offset:%24\n"
      "ds_read_b128 %11, %23 offset:%24\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6]), "v"(a[7]),
        "v"(a[8]), "v"(a[9]), "v"(a[10]), "v"(a[11]), "i"(IMM)
      : "memory");
}

// The lane's header and two qs pieces of the four blocks of a stage buffer:
// header of block b at hb + 2304 b, qs pieces at qb + 2304 b (+256).
__device__ __forceinline__ void lds_read_weights(uint32_t hb, uint32_t qb, u32x4 (&v)[12]) {
  asm volatile(
      "ds_read_b128 %0, %12\n"
      "ds_read_b128 %1, %13\n"
      "ds_read_b128 %2, %13 offset:256\n"
      "ds_read_b128 %3, %12 offset:2304\n"
      "ds_read_b128 %4, %13 offset:2304\n"
      "ds_read_b128 %5, %13 offset:2560\n"
      "ds_read_b128 %6, %12 offset:4608\n"
      "ds_read_b128 %7, %13 offset:4608\n"
      "ds_read_b128 %8, %13 offset:4864\n"
      "ds_read_b128 %9, %12 offset:6912\n"
      "ds_read_b128 %10, %13 offset:6912\n"
      "ds_read_b128 %11, %13 offset:7168\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11])
      : "v"(hb), "v"(qb)
      : "memory");
}

// The same for the two blocks of a two-block stage.
__device__ __forceinline__ void lds_read_weights2(uint32_t hb, uint32_t qb, u32x4 (&v)[6]) {
  asm volatile(
      "ds_read_b128 %0, %6\n"
      "ds_read_b128 %1, %7\n"
      "ds_read_b128 %2, %7 offset:256\n"
      "ds_read_b128 %3, %6 offset:2304\n"
      "ds_read_b128 %4, %7 offset:2304\n"
      "ds_read_b128 %5, %7 offset:2560\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
      : "v"(hb), "v"(qb)
      : "memory");
}

// Unit sums of the lane's two units in the four blocks (xb + 32 b), the
// four block exponents (eb) and their four side counts (one byte each, at
// eb + kCountOff).
__device__ __forceinline__ void lds_read_sums(uint32_t xb, uint32_t eb, u32x2 (&xs)[4], i32x4& ex,
                                              uint32_t& cnt) {
  static_assert(kCountOff == 512, "the offset below");
  asm volatile(
      "ds_read_b64 %0, %6\n"
      "ds_read_b64 %1, %6 offset:32\n"
      "ds_read_b64 %2, %6 offset:64\n"
      "ds_read_b64 %3, %6 offset:96\n"
      "ds_read_b128 %4, %7\n"
      "ds_read_b32 %5, %7 offset:512\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(xs[0]), "=&v"(xs[1]), "=&v"(xs[2]), "=&v"(xs[3]), "=&v"(ex), "=&v"(cnt)
      : "v"(xb), "v"(eb)
      : "memory");
}
// The same for the two blocks of a two-block stage (exponents in ex[0..1],
// the two side counts in the low 16 bits of cnt).
__device__ __forceinline__ void lds_read_sums2(uint32_t xb, uint32_t eb, u32x2 (&xs)[2], i32x4& ex,
                                               uint32_t& cnt) {
  static_assert(kCountOff == 512, "the offset below");
  u32x2 e2;
  asm volatile(
      "ds_read_b64 %0, %4\n"
      "ds_read_b64 %1, %4 offset:32\n"
      "ds_read_b64 %2, %5\n"
      "ds_read_u16 %3, %5 offset:512\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(xs[0]), "=&v"(xs[1]), "=&v"(e2), "=&v"(cnt)
      : "v"(xb), "v"(eb)
      : "memory");
  ex = i32x4{(int)e2[0], (int)e2[1], 0, 0};
}
// The 8 A images of two blocks (block b, MFMA t at addr + 1024 b + 256 t),
// read only by the lanes in `mask`; the other lanes keep their registers.
__device__ __forceinline__ void lds_read_images8(uint32_t addr, uint64_t mask, i32x4 (&a)[8]) {
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

__device__ __forceinline__ i32x4 low_nibbles(const u32x4& q) {
  return i32x4{(int)(q[0] & 0x0f0f0f0fu), (int)(q[1] & 0x0f0f0f0fu), (int)(q[2] & 0x0f0f0f0fu),
               (int)(q[3] & 0x0f0f0f0fu)};
}
__device__ __forceinline__ i32x4 high_nibbles(const u32x4& q) {
  return i32x4{(int)((q[0] >> 4) & 0x0f0f0f0fu), (int)((q[1] >> 4) & 0x0f0f0f0fu),
               (int)((q[2] >> 4) & 0x0f0f0f0fu), (int)((q[3] >> 4) & 0x0f0f0f0fu)};
}

// Exact value of a Q4_K/Q5_K weight with quant q of unit u (uniform) from
// the block's 16-byte header (d, dmin, the 12 scale bytes; quant.rs:176-185).
__device__ __forceinline__ float k4_weight(const u32x4& h, uint32_t u, uint32_t q) {
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const uint32_t sh = 8u * (u & 3u);
  const uint32_t sc = ((u < 4u ? sc03 : sc47) >> sh) & 0xffu;
  const uint32_t mn = ((u < 4u ? mn03 : mn47) >> sh) & 0xffu;
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  return k4_value_exact(__fmul_rn(d, (float)sc), __fmul_rn(dmin, (float)mn), q);
}

// Exact per-weight f32 dot of 16 nibbles (low or high half of each byte of q)
// with 16 activations.
__device__ __forceinline__ float exact_dot16(const u32x4& q, int shift, float d1, float m1,
                                             const float* __restrict__ xs, float acc) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t nib = (q[j >> 2] >> (8 * (j & 3) + shift)) & 0x0fu;
    acc = fmaf(k4_value_exact(d1, m1, nib), xs[j], acc);
  }
  return acc;
}

// One block of one lane's row, decoded once for every activation vector:
// B operands (low/high nibbles of its two qs pieces), the 6-bit scales and
// mins of units 2 grp, 2 grp + 1, d and dmin.
struct BlockQ4 {
  i32x4 la, ha, lb, hb;
  int sce, sco;
  float mne, mno, d, dmin;
};
__device__ __forceinline__ BlockQ4 decode_q4(const u32x4& h, const u32x4& qa, const u32x4& qb,
                                             bool hi_units, int bsh) {
  BlockQ4 w;
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const uint32_t scw = hi_units ? sc47 : sc03;
  const uint32_t mnw = hi_units ? mn47 : mn03;
  w.sce = (int)((scw >> bsh) & 0xffu);
  w.sco = (int)((scw >> (bsh + 8)) & 0xffu);
  w.mne = (float)((mnw >> bsh) & 0xffu);
  w.mno = (float)((mnw >> (bsh + 8)) & 0xffu);
  w.la = low_nibbles(qa);
  w.ha = high_nibbles(qa);
  w.lb = low_nibbles(qb);
  w.hb = high_nibbles(qb);
  w.d = half_bits_to_float(h[0] & 0xffffu);
  w.dmin = half_bits_to_float(h[0] >> 16);
  return w;
}

// Fast-path dot of one decoded block with one activation vector's images
// (xs: the fixed-point sums of the lane's two units); `err` gets the bound on
// its f32 rounding.  tc below is the exact integer sum_d T_d 256^d to within
// 5 * 2^-24 |tc| (a step of the fma chain rounds only when what is left of tc
// is far larger than the terms still to come), um = m_e X_e + m_o X_o to
// within 3 * 2^-24 (m_e |X_e| + m_o |X_o|), and the last fma rounds once:
// 2^-21 of the two terms' magnitudes covers all of it.
__device__ __forceinline__ float block_dot(const BlockQ4& w, const i32x4& a0, const i32x4& a1,
                                           const i32x4& a2, const i32x4& a3, u32x2 xs, int eb,
                                           float& err) {
  const i32x4 zero = {0, 0, 0, 0};
  i32x4 ce = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, w.la, zero, 0, 0, 0);
  i32x4 co = __builtin_amdgcn_mfma_i32_16x16x64_i8(a2, w.ha, zero, 0, 0, 0);
  ce = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, w.lb, ce, 0, 0, 0);
  co = __builtin_amdgcn_mfma_i32_16x16x64_i8(a3, w.hb, co, 0, 0, 0);
  const int t0 = __mul24(w.sce, ce[0]) + __mul24(w.sco, co[0]);
  const int t1 = __mul24(w.sce, ce[1]) + __mul24(w.sco, co[1]);
  const int t2 = __mul24(w.sce, ce[2]) + __mul24(w.sco, co[2]);
  const int t3 = __mul24(w.sce, ce[3]) + __mul24(w.sco, co[3]);
  const float tc =
      fmaf(fmaf(fmaf((float)t3, 256.0f, (float)t2), 256.0f, (float)t1), 256.0f, (float)t0);
  const float sxe = __uint_as_float(xs[0]), sxo = __uint_as_float(xs[1]);
  const float dt = w.d * tc;
  const float um = fmaf(w.mne, sxe, w.mno * sxo);
  const float ua = fmaf(w.mne, fabsf(sxe), w.mno * fabsf(sxo));
  err = __builtin_amdgcn_ldexpf(fmaf(fabsf(w.dmin), ua, fabsf(dt)), eb - 21);
  return __builtin_amdgcn_ldexpf(fmaf(-w.dmin, um, dt), eb);
}

// Exact per-weight path of one block (activations not finite or >= 2^100).
__device__ __forceinline__ float block_exact(const u32x4& h, const u32x4& qa, const u32x4& qb,
                                             bool hi_units, int bsh, const float* __restrict__ xs) {
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const uint32_t scw = hi_units ? sc47 : sc03;
  const uint32_t mnw = hi_units ? mn47 : mn03;
  const uint32_t sce = (scw >> bsh) & 0xffu, sco = (scw >> (bsh + 8)) & 0xffu;
  const uint32_t mne = (mnw >> bsh) & 0xffu, mno = (mnw >> (bsh + 8)) & 0xffu;
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  const float d1e = __fmul_rn(d, (float)sce), m1e = __fmul_rn(dmin, (float)mne);
  const float d1o = __fmul_rn(d, (float)sco), m1o = __fmul_rn(dmin, (float)mno);
  float acc = exact_dot16(qa, 0, d1e, m1e, xs, 0.0f);
  acc = exact_dot16(qb, 0, d1e, m1e, xs + 16, acc);
  acc = exact_dot16(qa, 4, d1o, m1o, xs + 32, acc);
  return exact_dot16(qb, 4, d1o, m1o, xs + 48, acc);
}

// Q5_K (quant.rs:67-125): the lane's header, the two qh pieces and its two qs
// pieces of the four blocks of a stage buffer -- block b's pieces start at
// hb + 2816 b (header, qh at +256, +512) and qb + 2816 b (qs, +256).
__device__ __forceinline__ void lds_read_weights5(uint32_t hb, uint32_t qb, u32x4 (&v)[20]) {
  asm volatile(
      "ds_read_b128 %0, %20\n"
      "ds_read_b128 %1, %20 offset:256\n"
      "ds_read_b128 %2, %20 offset:512\n"
      "ds_read_b128 %3, %21\n"
      "ds_read_b128 %4, %21 offset:256\n"
      "ds_read_b128 %5, %20 offset:2816\n"
      "ds_read_b128 %6, %20 offset:3072\n"
      "ds_read_b128 %7, %20 offset:3328\n"
      "ds_read_b128 %8, %21 offset:2816\n"
      "ds_read_b128 %9, %21 offset:3072\n"
      "ds_read_b128 %10, %20 offset:5632\n"
      "ds_read_b128 %11, %20 offset:5888\n"
      "ds_read_b128 %12, %20 offset:6144\n"
      "ds_read_b128 %13, %21 offset:5632\n"
      "ds_read_b128 %14, %21 offset:5888\n"
      "ds_read_b128 %15, %20 offset:8448\n"
      "ds_read_b128 %16, %20 offset:8704\n"
      "ds_read_b128 %17, %20 offset:8960\n"
      "ds_read_b128 %18, %21 offset:8448\n"
      "ds_read_b128 %19, %21 offset:8704\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(v[10]), "=&v"(v[11]),
        "=&v"(v[12]), "=&v"(v[13]), "=&v"(v[14]), "=&v"(v[15]), "=&v"(v[16]), "=&v"(v[17]),
        "=&v"(v[18]), "=&v"(v[19])
      : "v"(hb), "v"(qb)
      : "memory");
}

// The same for the two blocks of a two-block stage.
__device__ __forceinline__ void lds_read_weights5x2(uint32_t hb, uint32_t qb, u32x4 (&v)[10]) {
  asm volatile(
      "ds_read_b128 %0, %10\n"
      "ds_read_b128 %1, %10 offset:256\n"
      "ds_read_b128 %2, %10 offset:512\n"
      "ds_read_b128 %3, %11\n"
      "ds_read_b128 %4, %11 offset:256\n"
      "ds_read_b128 %5, %10 offset:2816\n"
      "ds_read_b128 %6, %10 offset:3072\n"
      "ds_read_b128 %7, %10 offset:3328\n"
      "ds_read_b128 %8, %11 offset:2816\n"
      "ds_read_b128 %9, %11 offset:3072\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
        "=&v"(v[6]), "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9])
      : "v"(hb), "v"(qb)
      : "memory");
}

// 5-bit weights of units 2 grp (low nibbles + qh bit 2 grp) and 2 grp + 1
// (high nibbles + bit 2 grp + 1) from 16 qs bytes and the matching 16 qh
// bytes.  rot_lo / rot_hi rotate that qh bit of every byte to bit 4
// (v_alignbit of a word with itself is a rotate right).
__device__ __forceinline__ void q5_operands(const u32x4& qs, const u32x4& qh, uint32_t rot_lo,
                                            uint32_t rot_hi, i32x4& lo, i32x4& hi) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t tl = __builtin_amdgcn_alignbit(qh[k], qh[k], rot_lo);
    const uint32_t th = __builtin_amdgcn_alignbit(qh[k], qh[k], rot_hi);
    lo[k] = (int)((qs[k] & 0x0f0f0f0fu) | (tl & 0x10101010u));
    hi[k] = (int)(((qs[k] >> 4) & 0x0f0f0f0fu) | (th & 0x10101010u));
  }
}

__device__ __forceinline__ BlockQ4 decode_q5(const u32x4& h, const u32x4& qh0, const u32x4& qh1,
                                             const u32x4& qa, const u32x4& qb, bool hi_units,
                                             int bsh, uint32_t rot_lo, uint32_t rot_hi) {
  BlockQ4 w = decode_q4(h, qa, qb, hi_units, bsh);  // scales, mins, d, dmin
  q5_operands(qa, qh0, rot_lo, rot_hi, w.la, w.ha);
  q5_operands(qb, qh1, rot_lo, rot_hi, w.lb, w.hb);
  return w;
}

// Exact per-weight f32 dot of 16 weights given as bytes (0..31) with 16
// activations.
__device__ __forceinline__ float exact_dot16_bytes(const i32x4& q, float d1, float m1,
                                                   const float* __restrict__ xs, float acc) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t v = ((uint32_t)q[j >> 2] >> (8 * (j & 3))) & 0xffu;
    acc = fmaf(k4_value_exact(d1, m1, v), xs[j], acc);
  }
  return acc;
}

// Exact per-weight path of one decoded Q5_K block (same element order as
// block_exact).
__device__ __forceinline__ float block_exact5(const BlockQ4& w, const u32x4& h, bool hi_units,
                                              int bsh, const float* __restrict__ xs) {
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const uint32_t scw = hi_units ? sc47 : sc03;
  const uint32_t mnw = hi_units ? mn47 : mn03;
  const uint32_t sce = (scw >> bsh) & 0xffu, sco = (scw >> (bsh + 8)) & 0xffu;
  const uint32_t mne = (mnw >> bsh) & 0xffu, mno = (mnw >> (bsh + 8)) & 0xffu;
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  const float d1e = __fmul_rn(d, (float)sce), m1e = __fmul_rn(dmin, (float)mne);
  const float d1o = __fmul_rn(d, (float)sco), m1o = __fmul_rn(dmin, (float)mno);
  float acc = exact_dot16_bytes(w.la, d1e, m1e, xs, 0.0f);
  acc = exact_dot16_bytes(w.lb, d1e, m1e, xs + 16, acc);
  acc = exact_dot16_bytes(w.ha, d1o, m1o, xs + 32, acc);
  return exact_dot16_bytes(w.hb, d1o, m1o, xs + 48, acc);
}

// Exact per-weight path of one decoded block (the order of block_exact):
// units 2 grp (la: elements 0..15, lb: 16..31 of the lane's 64) and
// 2 grp + 1 (ha, hb), quant.rs rounding.
__device__ __forceinline__ float block_exact_dec(const BlockQ4& w, const float* __restrict__ xs) {
  const float d1e = __fmul_rn(w.d, (float)w.sce), m1e = __fmul_rn(w.dmin, w.mne);
  const float d1o = __fmul_rn(w.d, (float)w.sco), m1o = __fmul_rn(w.dmin, w.mno);
  float acc = exact_dot16_bytes(w.la, d1e, m1e, xs, 0.0f);
  acc = exact_dot16_bytes(w.lb, d1e, m1e, xs + 16, acc);
  acc = exact_dot16_bytes(w.ha, d1o, m1o, xs + 32, acc);
  return exact_dot16_bytes(w.hb, d1o, m1o, xs + 48, acc);
}

// The weights of a stage of SB blocks in registers, per format: Q4_K keeps
// (header, qs piece a, qs piece b) per block, Q5_K adds the two qh pieces.
template <int QB, int SB = 4>
struct StageRegs {
  static constexpr int kPer = QB == 5 ? 5 : 3;
  u32x4 v[SB * kPer];
  __device__ __forceinline__ void read(uint32_t hb, uint32_t qb) {
    if constexpr (QB == 5 && SB == 4)
      lds_read_weights5(hb, qb, v);
    else if constexpr (QB == 5)
      lds_read_weights5x2(hb, qb, v);
    else if constexpr (SB == 4)
      lds_read_weights(hb, qb, v);
    else
      lds_read_weights2(hb, qb, v);
  }
  // a full-line stage buffer (Q4_K, four blocks): each piece at its own address
  template <int IMM>
  __device__ __forceinline__ void read_at(const uint32_t (&a)[12]) {
    static_assert(QB == 4 && SB == 4, "full-line stages: Q4_K, four blocks");
    lds_read_weights_at<IMM>(a, v);
  }
  __device__ __forceinline__ BlockQ4 decode(int b, bool hi_units, int bsh, uint32_t rot_lo,
                                            uint32_t rot_hi) const {
    if constexpr (QB == 5)
      return decode_q5(v[5 * b], v[5 * b + 1], v[5 * b + 2], v[5 * b + 3], v[5 * b + 4],
                       hi_units, bsh, rot_lo, rot_hi);
    else
      return decode_q4(v[3 * b], v[3 * b + 1], v[3 * b + 2], hi_units, bsh);
  }
  __device__ __forceinline__ float exact(int b, bool hi_units, int bsh, uint32_t rot_lo,
                                         uint32_t rot_hi, const float* __restrict__ xs) const {
    if constexpr (QB == 5)
      return block_exact5(decode(b, hi_units, bsh, rot_lo, rot_hi), v[5 * b], hi_units, bsh, xs);
    else
      return block_exact(v[3 * b], v[3 * b + 1], v[3 * b + 2], hi_units, bsh, xs);
  }
};

// Largest |w| of the lane's two units of a decoded Q4_K (QMAX 15) or Q5_K
// (QMAX 31) block: |d| sc QMAX + |dmin| m, the larger of the two units.
template <int QMAX>
__device__ __forceinline__ float k4_bound(const BlockQ4& w) {
  const float ad = fabsf(w.d), am = fabsf(w.dmin);
  return fmaxf(fmaf(ad, (float)(w.sce * QMAX), am * w.mne),
               fmaf(ad, (float)(w.sco * QMAX), am * w.mno));
}

// One vector's partial dot of the lane's row over stage s (blocks SB s ..
// SB s + nlive - 1), whose images and metadata sit at LDS stage ls: the MFMA
// digit sums, the rounded blocks' check (an exact recompute of them for a row
// that fails it), and the exact path for blocks that need it, summed over the
// lane groups
// (every lane of a row gets the row's sum).
template <int QB, int SB>
__device__ __forceinline__ float stage_rowsum(const StageRegs<QB, SB>& v, uint32_t sbase,
                                              const Layout& L, uint32_t ls, uint32_t s,
                                              uint32_t nlive, uint32_t grp, uint32_t n,
                                              i32x4 (&A)[8], bool hi_units, int bsh,
                                              uint32_t rot_lo, uint32_t rot_hi,
                                              const float* __restrict__ x) {
  static_assert(SB == 4 || SB == 2, "four- or two-block stages");
  u32x2 xs[SB];
  i32x4 ex;
  uint32_t cnt;
  if constexpr (SB == 4)
    lds_read_sums(sbase + L.xsum + 128u * ls + 8u * grp, sbase + L.expo + 16u * ls, xs, ex, cnt);
  else
    lds_read_sums2(sbase + L.xsum + 64u * ls + 8u * grp, sbase + L.expo + 8u * ls, xs, ex, cnt);
  float part[SB];
  float err = 0.0f;  // bound on the error of the fast-path partials
  bool bad_any = false;
#pragma unroll
  for (int h = 0; h < SB / 2; ++h) {
    lds_read_images8(sbase + L.img + 1024u * SB * ls + 2048u * h + 16u * n, kActiveLanes, A);
#pragma unroll
    for (int b2 = 0; b2 < 2; ++b2) {
      const int b = 2 * h + b2;
      const int eb = __builtin_amdgcn_readfirstlane(ex[b]);
      const bool use = (uint32_t)b < nlive;
      bad_any |= use && eb == kBadBlock;
      float e;
      const float c = block_dot(v.decode(b, hi_units, bsh, rot_lo, rot_hi), A[4 * b2],
                                A[4 * b2 + 1], A[4 * b2 + 2], A[4 * b2 + 3], xs[b], eb, e);
      const bool fast = use && eb != kBadBlock;
      part[b] = fast ? c : 0.0f;
      err += fast ? e : 0.0f;
    }
  }
  // the stage check (the factored form's rounding plus the rounded blocks'
  // bound); blocks on the exact path, and every live block of a row that
  // fails the check, take the per-weight path
  const uint32_t counts = live_counts(__builtin_amdgcn_readfirstlane(cnt), nlive);
  const uint32_t rmask = rounded_mask(counts);
  if (rmask != 0u) {
    const uint32_t list = sbase + L.expo + L.side_off + (uint32_t)SB * kSideBytes * ls;
    err += rounded_bound<SB>(list, rmask, grp, [&](auto b) {
      return k4_bound<QB == 5 ? 31 : 15>(
          v.decode(decltype(b)::value, hi_units, bsh, rot_lo, rot_hi));
    });
  }
  float apart = 0.0f;
#pragma unroll
  for (int b = 0; b < SB; ++b) apart += fabsf(part[b]);
  const uint32_t redo = stage_ok(err, apart) ? 0u : (1u << nlive) - 1u;
  if (bad_any || redo != 0u) {
#pragma unroll
    for (int b = 0; b < SB; ++b)
      if (((uint32_t)b < nlive && __builtin_amdgcn_readfirstlane(ex[b]) == kBadBlock) ||
          ((redo >> b) & 1u))
        part[b] = v.exact(b, hi_units, bsh, rot_lo, rot_hi,
                          x + 256u * ((uint32_t)SB * s + b) + 64u * grp);
  }
  if constexpr (SB == 4)
    return sum_lane_groups((part[0] + part[1]) + (part[2] + part[3]));
  else
    return sum_lane_groups(part[0] + part[1]);
}

// GROUPED: the rows are those of the group's matrices with one K, one after the
// other (every matrix but the last a whole number of 16-row tiles), and tile
// t's weights are those of the matrix whose tiles reach past t.
//
// SLICED (one matrix, one vector): a K-sliced launch (SliceArgs,
// mfma_common.h); the LDS holds the images and metadata of the workgroup's
// slice only, stage s of the matrix at local stage s - r_lo.
// SB (one matrix, one vector): blocks per stage, 4, or 2 for shapes whose
// workgroups have few pairs per wave (finer pairs, a shorter last one).
// LINES (Q4_K, one vector, four-block stages of whole rows, nb a multiple of
// 4, every matrix 128-byte aligned): full-line copies (kLineCopies above).
template <int WAVES, int DEPTH, int MATS, int NTOK, int QB, bool GROUPED, bool SLICED = false,
          int SB = 4, bool LINES = false>
__global__ __launch_bounds__(WAVES * 64) void q4k_matvec_mfma(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ w2,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, uint32_t rows,
                                                              uint32_t nb, void* __restrict__ wsp,
                                                              SchedArgs sa, GroupArgs ga,
                                                              SliceArgs sla) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  static_assert(NTOK == 1 || MATS == 1, "several activation vectors: one matrix");
  static_assert(QB == 4 || QB == 5, "Q4_K or Q5_K");
  static_assert(!SLICED || (MATS == 1 && NTOK == 1 && !GROUPED), "slices of one matrix and vector");
  static_assert(SB == 4 || (SB == 2 && MATS == 1 && NTOK == 1), "two-block stages: one vector");
  static_assert(!LINES || (QB == 4 && SB == 4 && NTOK == 1 && !SLICED && DEPTH <= 2),
                "full-line stages: Q4_K, four blocks, one vector, whole rows");
  if constexpr (GROUPED) load_group_args_early(ga);
  const uint32_t slots = sa.packed & 0xffu;
  // copy instructions per stage
  constexpr uint32_t kPieces = LINES ? kLineCopies : stage_copies(QB, SB);
  constexpr uint32_t kRowPieces = SB * block_pieces(QB);  // 16-byte pieces per row and stage
  constexpr uint32_t kStage = LINES ? kLineStage : stage_bytes(QB, SB);
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + SB - 1u) / SB;
  const uint32_t tstages = MATS * nstages;  // pairs (and partials) per tile
  // the schedule: whole and split tiles (sc), or K slices (ss)
  Sched sc{};
  SliceSched ss{};
  if constexpr (SLICED)
    ss = make_slice_sched(ntiles, sla, sa);
  else
    sc = make_sched(ntiles, tstages, WAVES, sa);
  // the stages whose images the LDS holds: from st0, nbl blocks
  const uint32_t st0 = SLICED ? ss.r_lo : 0u;
  const uint32_t nbl = SLICED ? min(SB * ss.ns, nb - SB * st0) : nb;
  const Layout L =
      layout(WAVES, DEPTH, SLICED ? SB * ss.pstride : nb, slots, MATS, NTOK, QB, SB, LINES);
  const SplitWs ws = split_ws(wsp);
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t row_bytes = nb * block_bytes(QB);
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  uint8_t* const wstage = smem + wave * DEPTH * kStage;

  // 1. x into the image area, natural order (block b at img + 1024 b; vector
  //    t of NTOK at img + t img_stride)
#pragma unroll
  for (int t = 0; t < NTOK; ++t)
    copy_x<WAVES>(smem, L.img + t * L.img_stride,
                  x + (size_t)t * nb * kBlockElems + (size_t)SB * st0 * kBlockElems, nbl, wave,
                  lane);

  // 2. this wave's pairs k = wave, wave + WAVES, ... of the workgroup's pairs
  //    (pair_at: a tile and its partial r, r being stage r % nstages of
  //    matrix r / nstages), and the copies of its first DEPTH, pair j of the
  //    wave into buffer j % DEPTH.  Piece
  //    c = 64 i + lane of a stage is piece c / 16 of row c % 16's 576 bytes.
  auto pair_of = [&](uint32_t k) -> Pair {
    if constexpr (SLICED)
      return pair_at(ss, k);
    else
      return pair_at(sc, k, tstages);
  };
  const uint32_t npairs = SLICED ? ss.npairs : sc.npairs;
  const uint32_t voff = n * row_bytes + 16u * grp;
  // LINES: lcopy0 / lcopy1, the copy lane's byte offset in its tile for rows
  // 2 i and 2 i + 1 before 576 s - 64 m (the row's stage starts 64 m bytes
  // into its first line, m = c ^ parity of the stage).
  uint32_t lcopy0 = 0u, lcopy1 = 0u;
  if constexpr (LINES) {
    const uint32_t li = lane >> 3, k = ((lane & 7u) - (li >> 1)) & 7u;
    lcopy0 = 2u * li * row_bytes + 16u * k;
    lcopy1 = lcopy0 + row_bytes;
  }
  const uint32_t my_pairs = wave < npairs ? (npairs - 1u - wave) / WAVES + 1u : 0u;
  auto issue = [&](uint32_t j, const Pair& pr) {
    const uint32_t mat = MATS > 1 && pr.r >= nstages ? 1u : 0u, st = pr.r - mat * nstages;
    uint32_t row0 = pr.tile * 16u, mrows = rows;
    const uint8_t* wm = mat ? w2 : w;
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
    const uint32_t nrows = min(16u, mrows - row0);
    if constexpr (LINES) {
      // the tile's rows from its first byte (128-byte aligned); rows past
      // the tile's last read zero
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(wm + (size_t)row0 * row_bytes), 0, (int)(nrows * row_bytes),
          kBufferWord3);
      uint8_t* dst = wstage + (j % DEPTH) * kStage;
      const uint32_t odd = st & 1u;
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        // (the stage's terms are uniform: one add per copy class)
        const uint32_t vo =
            (c ? lcopy1 : lcopy0) + (4u * kQ4Bytes * st - 64u * ((uint32_t)c ^ odd));
        uint8_t* const region = dst + 1024u * ((uint32_t)c ^ odd);
        // (the line's offset goes into the lane offset: an instruction offset
        // would move the LDS destination by the same amount)
#pragma unroll
        for (int jl = 0; jl < 5; ++jl)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(region + 2048 * jl), 16,
                                                    vo + 128u * jl, 0, 0, kNontemporal);
      }
      return;
    }
    const uint8_t* sb = wm + (size_t)row0 * row_bytes + SB * block_bytes(QB) * st;
    // the descriptor ends at the tile's last row: pieces past it read zero
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - SB * block_bytes(QB) * st),
        kBufferWord3);
    uint8_t* dst = wstage + (j % DEPTH) * kStage;
#pragma unroll
    for (int i = 0; i < (int)kPieces; ++i) {
      // (a stage of SB = 2 ends inside its last copy: those lanes re-read the
      // row's last piece, which adds no traffic)
      const uint32_t off = 4u * (uint32_t)i + 3u < kRowPieces
                               ? voff + 64u * i
                               : n * row_bytes + 16u * min(4u * i + grp, kRowPieces - 1u);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst + 1024 * i), 16, off, 0, 0, 0);
    }
  };
  // (with one stage in flight, the pair of the next stage, worked out when
  // its copy is issued, is kept for its turn)
  Pair pr_next = pair_of(wave);
  auto issue_first = [&]() {
#pragma unroll
    for (int j = 0; j < DEPTH; ++j)
      if ((uint32_t)j < my_pairs) issue(j, j == 0 ? pr_next : pair_of(wave + j * WAVES));
  };

  // 3. ring slots and the builders' count, set before any wave goes on (the
  //    waves start together, so this barrier costs little).  The first round
  //    of waves (one per SIMD, and every builder), whose copies the empty
  //    memory queue takes at once, issue their first copies before it; the
  //    later waves, whose copies the queue holds back, after it, so that none
  //    of them keeps the others at the barrier.  A builder that issued late
  //    would hold every wave's first arithmetic back with its images.  The
  //    waves that copied x (the builders) turn it
  //    into digit images, unit sums and exponents once it has landed (the
  //    copies complete in issue order).  A wave reads images only once every
  //    builder has counted itself done (wait_images): no barrier makes a
  //    wave whose stage has landed wait for the waves whose copies the
  //    memory queue still holds back.
  const bool first_round = wave < max(4u, min((uint32_t)WAVES, (nbl + 3u) / 4u));
  if (first_round) issue_first();
  init_slots<WAVES>(sbase, L, slots);
  lds_wait();
  __builtin_amdgcn_s_barrier();
  const uint32_t builders = min((uint32_t)WAVES, (nbl + 3u) / 4u);
  if (!first_round) issue_first();
  if (wave < builders) {
    const uint32_t early = min((uint32_t)DEPTH, my_pairs);
    if (early >= 3u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(3 * kPieces));
    else if (early == 2u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kPieces));
    else if (early == 1u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kPieces));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    // chunk c = 4 p + t: units 2p, 2p + 1 of lane group p, MFMA t
#pragma unroll
    for (int t = 0; t < NTOK; ++t)
      build_images<WAVES>(sbase, L, nbl, wave, grp, n,
                          [](uint32_t c) { return 256u * (c & 3u) + 64u * (c >> 2); }, t);
    lds_wait();
    if (lane == 0u) (void)lds_add_rtn(sbase + L.ready, 1u);
  }

  // 4. the wave's pairs
  const bool hi_units = grp >= 2u;       // units 4..7 use the packed upper scales
  const int bsh = 16 * (int)(grp & 1u);  // byte of unit 2 grp within its scale word
  const uint32_t hb0 = sbase + wave * DEPTH * kStage + 16u * n;
  // qs pieces of lane group grp: Q4_K pieces 1 + 2 grp, Q5_K 3 + 2 grp
  const uint32_t qb0 = hb0 + (QB == 5 ? 768u : 256u) + 512u * grp;
  // Q5_K: rotations that bring qh bits 2 grp / 2 grp + 1 of each byte to bit 4
  const uint32_t rot_lo = (28u + 2u * grp) & 31u, rot_hi = (29u + 2u * grp) & 31u;
  // the images of two blocks at a time: the lanes that do not read them keep
  // zeros, so the registers stay live through the loop (32 rather than 64)
  i32x4 A[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) A[t] = i32x4{0, 0, 0, 0};
  // LINES: the lane's 12 pieces of a stage in buffer 0 (the header, qs
  // pieces 1 + 2 grp and 2 + 2 grp of each block), the same at every stage:
  // the lane's row (n, or n ^ 1 in odd stages) starts its stage 64 m bytes
  // into its first line, m = n & 1, so piece q sits at position q + 4 m of
  // the row's five lines, line j = pos / 8 in LDS region 2 j + (n & 1), slot
  // 8 (n >> 1) + ((pos + (n >> 2)) & 7).
  uint32_t lread[12];
  if constexpr (LINES) {
    const uint32_t ri = n >> 1, rc = n & 1u, phi = n >> 2;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
#pragma unroll
      for (int pc = 0; pc < 3; ++pc) {
        const uint32_t q = 9u * b + (pc == 0 ? 0u : (uint32_t)pc + 2u * grp);
        const uint32_t pos = q + 4u * rc;
        lread[3 * b + pc] = sbase + wave * DEPTH * kStage + 1024u * (2u * (pos >> 3) + rc) +
                            128u * ri + 16u * (((pos & 7u) + phi) & 7u);
      }
    }
  }
  uint32_t fail = 0u;  // a bounded wait that gave up (kDevErr*)
  bool images = false;  // every builder's images seen done
  // The fused gate/up (two matrices) with one stage in flight and three or
  // more pairs per wave: a wave claims the workgroup's pairs after its first
  // (pair `wave`) from a counter (L.ready + 4) as it issues their copies, so
  // the waves whose first copies went out late take fewer pairs instead of
  // finishing after the rest (17408 x 5120, 42 pairs per workgroup: 20.9 ->
  // 19.3 us).  With fewer pairs per wave an early wave would take a third
  // pair and end a whole pair later (the 17408 x 5120 matvec, 21 pairs per
  // workgroup: 11.2 -> 12.7 us), and in one-matrix kernels the claim's code
  // alone cost the headline 0.13 us, so there wave w takes pairs w,
  // w + WAVES, ...  Which wave computes a pair changes no sum: a tile's
  // finishing wave adds its partials in order.
  constexpr bool kClaimable = DEPTH == 1 && MATS == 2;
  const bool claims = kClaimable && npairs >= 3u * (uint32_t)WAVES;
  uint32_t knext = wave;  // claims: the index of pr_next
  for (uint32_t j = 0; claims ? knext < npairs : j < my_pairs; ++j) {
    const Pair pr = DEPTH == 1 ? pr_next : pair_of(wave + j * WAVES);
    const uint32_t s = MATS > 1 && pr.r >= nstages ? pr.r - nstages : pr.r;  // stage
    const uint32_t later = min((uint32_t)DEPTH - 1u, my_pairs - 1u - j);
    if (DEPTH >= 3 && later >= 2u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kPieces));
    else if (DEPTH >= 2 && later >= 1u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kPieces));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const uint32_t buf = (j % DEPTH) * kStage;
    StageRegs<QB, SB> v;
    if constexpr (LINES) {
      if (DEPTH > 1 && (j & 1u) != 0u)
        v.template read_at<(int)kLineStage>(lread);
      else
        v.template read_at<0>(lread);
    } else {
      v.read(hb0 + buf, qb0 + buf);
    }
    // The buffer just read is free again.  With one vector its next copy
    // goes out after the stage's arithmetic: while the memory queue is full,
    // issuing a copy holds the wave, and the stage in registers would wait
    // for it.
    auto issue_next = [&]() {
      if (kClaimable && claims) {
        knext = lds_claim(sbase + L.ready + 4u);
        if (knext < npairs) {
          const Pair pn = pair_of(knext);
          issue(0u, pn);
          pr_next = pn;
        }
      } else if (j + DEPTH < my_pairs) {
        const Pair pn = pair_of(wave + (j + DEPTH) * WAVES);
        issue(j + DEPTH, pn);
        if (DEPTH == 1) pr_next = pn;
      }
    };
    if (NTOK > 1) issue_next();
    const uint32_t nlive = min((uint32_t)SB, nb - SB * s);
    if (!images) {
      wait_images(sbase, L, builders, fail);
      images = true;
    }
    if constexpr (NTOK > 1) {
      // the stage's weights are decoded once and meet every vector in turn
      BlockQ4 bw[4];
#pragma unroll
      for (int b = 0; b < 4; ++b)
        bw[b] = v.decode(b, hi_units, bsh, rot_lo, rot_hi);
      float rs[NTOK];
#pragma unroll
      for (int t = 0; t < NTOK; ++t) {
        u32x2 xs[4];
        i32x4 ex;
        uint32_t cnt;
        lds_read_sums(sbase + L.xsum + t * L.xsum_stride + 128u * s + 8u * grp,
                      sbase + L.expo + t * L.expo_stride + 16u * s, xs, ex, cnt);
        float part[4];
        float err = 0.0f;
        bool bad_any = false;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          lds_read_images8(sbase + L.img + t * L.img_stride + 4096u * s + 2048u * h + 16u * n,
                           kActiveLanes, A);
#pragma unroll
          for (int b2 = 0; b2 < 2; ++b2) {
            const int b = 2 * h + b2;
            const int eb = __builtin_amdgcn_readfirstlane(ex[b]);
            const bool use = (uint32_t)b < nlive;
            bad_any |= use && eb == kBadBlock;
            float e;
            const float c = block_dot(bw[b], A[4 * b2], A[4 * b2 + 1], A[4 * b2 + 2],
                                      A[4 * b2 + 3], xs[b], eb, e);
            const bool fast = use && eb != kBadBlock;
            part[b] = fast ? c : 0.0f;
            err += fast ? e : 0.0f;
          }
        }
        const uint32_t counts = live_counts(__builtin_amdgcn_readfirstlane(cnt), nlive);
        const uint32_t rmask = rounded_mask(counts);
        if (rmask != 0u) {
          const uint32_t list =
              sbase + L.expo + t * L.expo_stride + L.side_off + 4u * kSideBytes * s;
          err += rounded_bound<4>(list, rmask, grp, [&](auto b) {
            return k4_bound<QB == 5 ? 31 : 15>(bw[decltype(b)::value]);
          });
        }
        const float apart = (fabsf(part[0]) + fabsf(part[1])) + (fabsf(part[2]) + fabsf(part[3]));
        const uint32_t redo = stage_ok(err, apart) ? 0u : (1u << nlive) - 1u;
        if (bad_any || redo != 0u) {
#pragma unroll
          for (int b = 0; b < 4; ++b)
            if (((uint32_t)b < nlive && __builtin_amdgcn_readfirstlane(ex[b]) == kBadBlock) ||
                ((redo >> b) & 1u))
              part[b] = block_exact_dec(
                  bw[b], x + (size_t)t * nb * kBlockElems + 256u * (4u * s + b) + 64u * grp);
        }
        rs[t] = sum_lane_groups((part[0] + part[1]) + (part[2] + part[3]));
      }
      hand_off_tokens<NTOK>(sbase, L, sc.by_slots, pr, tstages, rs, lane, rows, y, fail);
      continue;
    }
    float rowsum = stage_rowsum(v, sbase, L, s - st0, s, nlive, grp, n, A, hi_units, bsh,
                                rot_lo, rot_hi, x);
    // LINES: in odd stages lane n summed row n ^ 1; swap adjacent lanes back
    if (LINES && (s & 1u) != 0u) rowsum = dpp<kQuadSwap>(rowsum);
    issue_next();

    // hand the 16 row partials to the tile's slot; the last stage finishes it
    if constexpr (SLICED)
      hand_off_slice(sbase, L, ss, pr, rowsum, lane, rows, y, ws, fail);
    else
      hand_off<MATS>(sbase, L, slots, sc, sa, pr, nstages, rowsum, lane, rows, y, ws, fail);
  }
  if (fail != 0u) report_device_error(wsp, fail);
}

// ---- Several activation vectors in the MFMA rows --------------------------
//
// For a pass over the weights with 2..4 activation vectors (matmul-many,
// replacing si_q4_k_matmul_many, metal.rs:1052-1262) the vectors share the A
// operand of v_mfma_i32_16x16x32_i8, whose K = 32 is exactly one unit:
//
//  * A row 4 t + d holds digit d of vector t over the unit's 32 activations
//    (lane 16 g + m supplies activations 8 g .. 8 g + 7 of row m); vectors
//    past the pass's count are zero.
//  * B lane (g, n) holds weights 8 g .. 8 g + 7 of the unit for tile row n:
//    the low (unit 2 j) or high (unit 2 j + 1) nibbles of qs bytes
//    32 j + 8 g .. 32 j + 8 g + 7.
//  * Result lane (g, n) holds the four digit sums of vector g and row n, so
//    T_d = sum_u sc_u C_u[d] over the block's eight units and the row's dot
//    stay in that lane: y_g[n] += d * (sum_d T_d 256^d) * 2^(e_gb - 30) -
//    dmin * sum_u m_u X_gu, with X_gu the f32 sum of vector g's unit u.
//
// Group images (4 KB per block, in the place of the four vectors' copies):
// block b at img + 4096 b, unit pair p at + 1024 p, lane l at + 16 l, units
// 2 p and 2 p + 1 in its two 8-byte halves.
//
// K slices.  Four vectors' images of a whole row (4 KB per block) would
// crowd the stage buffers out of LDS, and with them the bytes in flight.  So
// a launch with S > 1 cuts K into its S stages: GS workgroups per stage,
// workgroup g works on stage k = g / GS for tiles g % GS, g % GS + GS, ...,
// and keeps the images of that stage only.  Each pair is then its
// workgroup's whole share of a tile: the wave stores each vector's and row's
// sum over the stage in the scratch (part_out[(k * 4 NG + v) * rows + row],
// or kPartRedo for a stage left to the exact path), and tok_reduce adds the
// S sums in stage order (deterministic).  With S == 1 a workgroup keeps the
// whole row's images and sums a tile's stages in its LDS slot ring.

// Headers and the lane's four 8-byte qs slices of the four blocks of a stage
// buffer: header of block b at hb + 2304 b, slice j at qb + 2304 b + 512 j.
__device__ __forceinline__ void lds_read_weights_tok4(uint32_t hb, uint32_t qb, u32x4 (&h)[4],
                                                      u32x2 (&q)[16]) {
  asm volatile(
      "ds_read_b128 %0, %20\n"
      "ds_read_b64 %4, %21\n"
      "ds_read_b64 %5, %21 offset:512\n"
      "ds_read_b64 %6, %21 offset:1024\n"
      "ds_read_b64 %7, %21 offset:1536\n"
      "ds_read_b128 %1, %20 offset:2304\n"
      "ds_read_b64 %8, %21 offset:2304\n"
      "ds_read_b64 %9, %21 offset:2816\n"
      "ds_read_b64 %10, %21 offset:3328\n"
      "ds_read_b64 %11, %21 offset:3840\n"
      "ds_read_b128 %2, %20 offset:4608\n"
      "ds_read_b64 %12, %21 offset:4608\n"
      "ds_read_b64 %13, %21 offset:5120\n"
      "ds_read_b64 %14, %21 offset:5632\n"
      "ds_read_b64 %15, %21 offset:6144\n"
      "ds_read_b128 %3, %20 offset:6912\n"
      "ds_read_b64 %16, %21 offset:6912\n"
      "ds_read_b64 %17, %21 offset:7424\n"
      "ds_read_b64 %18, %21 offset:7936\n"
      "ds_read_b64 %19, %21 offset:8448\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(q[0]), "=&v"(q[1]),
        "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]), "=&v"(q[7]),
        "=&v"(q[8]), "=&v"(q[9]), "=&v"(q[10]), "=&v"(q[11]), "=&v"(q[12]), "=&v"(q[13]),
        "=&v"(q[14]), "=&v"(q[15])
      : "v"(hb), "v"(qb)
      : "memory");
}

// Q5_K (176-byte blocks: header, qh at +16, qs at +48): the same for a stage
// buffer of Q5_K blocks -- header of block b at hb + 2816 b, qs slice j at
// qb + 2816 b + 512 j -- and the lane's 8-byte qh slice of each block (the qh
// bytes of its elements 8 g .. 8 g + 7, bit u for unit u) at qhb + 2816 b.
__device__ __forceinline__ void lds_read_weights_tok5(uint32_t hb, uint32_t qb, uint32_t qhb,
                                                      u32x4 (&h)[4], u32x2 (&q)[16],
                                                      u32x2 (&qh)[4]) {
  asm volatile(
      "ds_read_b128 %0, %24\n"
      "ds_read_b64 %4, %25\n"
      "ds_read_b64 %5, %25 offset:512\n"
      "ds_read_b64 %6, %25 offset:1024\n"
      "ds_read_b64 %7, %25 offset:1536\n"
      "ds_read_b64 %20, %26\n"
      "ds_read_b128 %1, %24 offset:2816\n"
      "ds_read_b64 %8, %25 offset:2816\n"
      "ds_read_b64 %9, %25 offset:3328\n"
      "ds_read_b64 %10, %25 offset:3840\n"
      "ds_read_b64 %11, %25 offset:4352\n"
      "ds_read_b64 %21, %26 offset:2816\n"
      "ds_read_b128 %2, %24 offset:5632\n"
      "ds_read_b64 %12, %25 offset:5632\n"
      "ds_read_b64 %13, %25 offset:6144\n"
      "ds_read_b64 %14, %25 offset:6656\n"
      "ds_read_b64 %15, %25 offset:7168\n"
      "ds_read_b64 %22, %26 offset:5632\n"
      "ds_read_b128 %3, %24 offset:8448\n"
      "ds_read_b64 %16, %25 offset:8448\n"
      "ds_read_b64 %17, %25 offset:8960\n"
      "ds_read_b64 %18, %25 offset:9472\n"
      "ds_read_b64 %19, %25 offset:9984\n"
      "ds_read_b64 %23, %26 offset:8448\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(q[0]), "=&v"(q[1]),
        "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]), "=&v"(q[7]),
        "=&v"(q[8]), "=&v"(q[9]), "=&v"(q[10]), "=&v"(q[11]), "=&v"(q[12]), "=&v"(q[13]),
        "=&v"(q[14]), "=&v"(q[15]), "=&v"(qh[0]), "=&v"(qh[1]), "=&v"(qh[2]), "=&v"(qh[3])
      : "v"(hb), "v"(qb), "v"(qhb)
      : "memory");
}

// The stage of a vectors-in-rows pass in registers: per block its header,
// the lane's four 8-byte qs slices and (Q5_K) its qh slice.
template <int QB>
struct TokStage {
  u32x4 h[4];
  u32x2 q[16];
  u32x2 qh[QB == 5 ? 4 : 1];
};
// The lane's stage addresses: header (hb0), qs slices (qb0) and qh slice
// (qhb0, Q5_K) of the stage's first block.
struct TokAddr {
  uint32_t hb0, qb0, qhb0;
};
template <int QB>
__device__ __forceinline__ void lds_read_weights_tok(const TokAddr& a, TokStage<QB>& st) {
  if constexpr (QB == 5)
    lds_read_weights_tok5(a.hb0, a.qb0, a.qhb0, st.h, st.q, st.qh);
  else
    lds_read_weights_tok4(a.hb0, a.qb0, st.h, st.q);
}

// The lane's group-image quarters of one block (unit pairs 0..3) and its
// vector's eight unit sums.
__device__ __forceinline__ void lds_read_group_block(uint32_t ia, uint32_t xa, u32x4 (&a)[4],
                                                     u32x4 (&xs)[2]) {
  asm volatile(
      "ds_read_b128 %0, %6\n"
      "ds_read_b128 %1, %6 offset:1024\n"
      "ds_read_b128 %2, %6 offset:2048\n"
      "ds_read_b128 %3, %6 offset:3072\n"
      "ds_read_b128 %4, %7\n"
      "ds_read_b128 %5, %7 offset:16\n"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(xs[0]), "=&v"(xs[1])
      : "v"(ia), "v"(xa)
      : "memory");
}

// The eight MFMAs of one block of row n against the lane's vector: c[u] the
// four digit sums of unit u.  Q5_K: bit u of each qh byte is the weight's
// fifth bit (rotated to bit 4: v_alignbit of a word with itself).
template <int QB>
__device__ __forceinline__ void block_mfma_tok(const TokStage<QB>& st, int b,
                                               const u32x4 (&a)[4], i32x4 (&c)[8]) {
  const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const u32x2 w = st.q[4 * b + j];
    uint32_t lo0 = w[0] & 0x0f0f0f0fu, lo1 = w[1] & 0x0f0f0f0fu;
    uint32_t hi0 = (w[0] >> 4) & 0x0f0f0f0fu, hi1 = (w[1] >> 4) & 0x0f0f0f0fu;
    if constexpr (QB == 5) {
      const u32x2 qh = st.qh[b];
      const uint32_t rl = (2u * j + 28u) & 31u, rh = (2u * j + 29u) & 31u;  // bit u -> bit 4
      lo0 |= __builtin_amdgcn_alignbit(qh[0], qh[0], rl) & 0x10101010u;
      lo1 |= __builtin_amdgcn_alignbit(qh[1], qh[1], rl) & 0x10101010u;
      hi0 |= __builtin_amdgcn_alignbit(qh[0], qh[0], rh) & 0x10101010u;
      hi1 |= __builtin_amdgcn_alignbit(qh[1], qh[1], rh) & 0x10101010u;
    }
    c[2 * j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_i64(a[j][0], a[j][1]), as_i64(lo0, lo1),
                                                     zero, 0, 0, 0);
    c[2 * j + 1] = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_i64(a[j][2], a[j][3]),
                                                         as_i64(hi0, hi1), zero, 0, 0, 0);
  }
}

// One block of row n against vector g (the lane's), fast path: eight MFMAs,
// the integer scale combine and the f32 digit and min terms over the
// fixed-point unit sums xs; `err` gets the bound on its f32 rounding.  The
// eight-term um is summed in pairs (within 5 * 2^-24 sum_u m_u |X_u| with the
// sums' own rounding), so as in block_dot 2^-21 of the two terms' magnitudes
// covers the whole.
template <int QB>
__device__ __forceinline__ float block_dot_tok(const TokStage<QB>& st, int b,
                                               const u32x4 (&a)[4], const u32x4 (&xs)[2], int eb,
                                               float& err) {
  const u32x4 h = st.h[b];
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  i32x4 c[8];
  block_mfma_tok<QB>(st, b, a, c);
  int t[4] = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int s = (int)(((u < 4 ? sc03 : sc47) >> (8 * (u & 3))) & 0xffu);
#pragma unroll
    for (int d = 0; d < 4; ++d) t[d] = mad_i24(s, c[u][d], t[d]);
  }
  const float tc =
      fmaf(fmaf(fmaf((float)t[3], 256.0f, (float)t[2]), 256.0f, (float)t[1]), 256.0f, (float)t[0]);
  float pr[4], ua = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int u = 2 * k;
    const float m0 = (float)(((u < 4 ? mn03 : mn47) >> (8 * (u & 3))) & 0xffu);
    const float m1 = (float)(((u < 4 ? mn03 : mn47) >> (8 * ((u + 1) & 3))) & 0xffu);
    const float s0 = __uint_as_float(xs[u >> 2][u & 3]);
    const float s1 = __uint_as_float(xs[u >> 2][(u + 1) & 3]);
    pr[k] = fmaf(m1, s1, m0 * s0);
    ua = fmaf(m1, fabsf(s1), fmaf(m0, fabsf(s0), ua));
  }
  const float um = (pr[0] + pr[1]) + (pr[2] + pr[3]);
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  const float dt = d * tc;
  err = __builtin_amdgcn_ldexpf(fmaf(fabsf(dmin), ua, fabsf(dt)), eb - 21);
  return __builtin_amdgcn_ldexpf(fmaf(-dmin, um, dt), eb);
}

// block_dot_tok's second try for a lane whose stage failed its check: the
// same eight MFMAs and the same int32 digit sums T_d = sum_u sc_u C_u[d], then
// sum_d 256^d T_d (< 2^50) formed exactly in f64 and the min term's products
// (exact in f64) summed in f64.  What rounding is
// left is that of the f32 unit sums xs (2^-24 each) and the f64 steps, so
// err = 2^(eb-24) 1.01 |dmin| sum_u m_u |xs_u| + 2^(eb-48) of the two terms,
// about an eighth of the fast path's bound.
template <int QB>
__device__ __forceinline__ double block_dot_tok_f64(const TokStage<QB>& st, int b,
                                                    const u32x4 (&a)[4], const u32x4 (&xs)[2],
                                                    int eb, float& err) {
  const u32x4 h = st.h[b];
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  i32x4 c[8];
  block_mfma_tok<QB>(st, b, a, c);
  int t[4] = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int s = (int)(((u < 4 ? sc03 : sc47) >> (8 * (u & 3))) & 0xffu);
#pragma unroll
    for (int d = 0; d < 4; ++d) t[d] = mad_i24(s, c[u][d], t[d]);
  }
  const double tc =
      fma(fma(fma((double)t[3], 256.0, (double)t[2]), 256.0, (double)t[1]), 256.0, (double)t[0]);
  double um = 0.0, ua = 0.0;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const double mn = (double)((((u < 4 ? mn03 : mn47) >> (8 * (u & 3))) & 0xffu));
    const double xu = (double)__uint_as_float(xs[u >> 2][u & 3]);
    um = fma(mn, xu, um);
    ua = fma(mn, fabs(xu), ua);
  }
  const double d = (double)half_bits_to_float(h[0] & 0xffffu);
  const double dmin = (double)half_bits_to_float(h[0] >> 16);
  const double dt = d * tc;
  const double mt = fabs(dmin) * ua;
  err = (float)ldexp(fma(0x1.02p-24, mt, 0x1p-48 * (fabs(dt) + mt)), eb);
  return ldexp(fma(-dmin, um, dt), eb);
}

// Exact per-weight path of one block of row n against 256 activations: the
// block's 144 (Q4_K) or 176 (Q5_K) bytes at byte `off` of the buffer `wr`
// (read from memory: by then the stage buffer may hold the next stage; bytes
// past the buffer's end, those of rows past the matrix, read as zero).
__device__ __forceinline__ float block_exact_row5(__amdgpu_buffer_rsrc_t wr, uint32_t off,
                                                  const float* __restrict__ xs);
template <int QB>
__device__ __forceinline__ float block_exact_row(__amdgpu_buffer_rsrc_t wr, uint32_t off,
                                                 const float* __restrict__ xs) {
  if constexpr (QB == 5) return block_exact_row5(wr, off, xs);
  auto ld = [&](uint32_t o) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off + o, 0, 0));
  };
  const u32x4 h = ld(0u);
  u32x4 qa[4], qb[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    qa[k] = ld(16u + 16u * k);
    qb[k] = ld(80u + 16u * k);
  }
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    // unit u: the low (even u) or high nibbles of qs pieces u & ~1, (u & ~1) + 1
    const uint32_t sc = ((u < 4 ? sc03 : sc47) >> (8 * (u & 3))) & 0xffu;
    const uint32_t mn = ((u < 4 ? mn03 : mn47) >> (8 * (u & 3))) & 0xffu;
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
    const int shift = 4 * (u & 1);
    const int k = u & ~1;
    acc = exact_dot16(k < 4 ? qa[k] : qb[k - 4], shift, d1, m1, xs + 32 * u, acc);
    acc = exact_dot16(k < 4 ? qa[k + 1] : qb[k - 3], shift, d1, m1, xs + 32 * u + 16, acc);
  }
  return acc;
}

// Q5_K: unit u of the block is the low (even u) or high nibbles of qs bytes
// 32 (u / 2) .. + 31 (at 48) with bit u of qh bytes 0 .. 31 (at 16) as the
// fifth bit (quant.rs:67-125); the same order as the Q4_K form.
__device__ __forceinline__ float block_exact_row5(__amdgpu_buffer_rsrc_t wr, uint32_t off,
                                                  const float* __restrict__ xs) {
  auto ld = [&](uint32_t o) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, off + o, 0, 0));
  };
  const u32x4 h = ld(0u);
  const u32x4 qh[2] = {ld(16u), ld(32u)};
  u32x4 qs[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) qs[k] = ld(48u + 16u * k);
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const float d = half_bits_to_float(h[0] & 0xffffu);
  const float dmin = half_bits_to_float(h[0] >> 16);
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint32_t sc = ((u < 4 ? sc03 : sc47) >> (8 * (u & 3))) & 0xffu;
    const uint32_t mn = ((u < 4 ? mn03 : mn47) >> (8 * (u & 3))) & 0xffu;
    const float d1 = __fmul_rn(d, (float)sc), m1 = __fmul_rn(dmin, (float)mn);
    const int shift = 4 * (u & 1);
    const int k = u & ~1;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const u32x4 q = qs[k + half], hbits = qh[half];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t wq = ((q[j >> 2] >> (8 * (j & 3) + shift)) & 0x0fu) |
                            (((hbits[j >> 2] >> (8 * (j & 3) + u)) & 1u) << 4);
        acc = fmaf(k4_value_exact(d1, m1, wq), xs[32 * u + 16 * half + j], acc);
      }
    }
  }
  return acc;
}

// Launch constants: the slice count S (1: whole rows), GS workgroups per
// slice (all of them when S == 1), the ring's slot count, and the division
// constants of GS, of the stages per tile and of the slot count.
struct TokArgs {
  uint32_t slices, groups_per_slice, m_gps, m_parts;
  uint32_t slots, m_slots;
  void* wsp;  // the workspace, for failure reports
};

// LDS map: per-wave stage buffers; the images of ng groups of nbl blocks
// (4 ng vectors), their unit sums and exponents; the slot ring (unused with
// K slices).
template <int QB>
__host__ __device__ constexpr Layout tok_layout(uint32_t waves, uint32_t nbl, uint32_t ng,
                                                uint32_t slots) {
  return make_layout(stage_bytes(QB), 4u, 32u, waves, 1u, nbl, slots, 1u, 4u * ng);
}

// One vector group's sum over the live blocks of a stage (the weights in h,
// q) on the fast path; blocks of the lane's vector that must take the exact
// path count zero here.  iabase/xabase/eabase: the group's images, the
// vector's unit sums and exponents at the stage's first block.  abs_part and
// err get the lane's sum of |block dot| and the bound on their rounding.
template <int QB>
__device__ __forceinline__ float tok_group_stage(const TokStage<QB>& st, uint32_t nlive,
                                                 uint32_t iabase, uint32_t xabase,
                                                 uint32_t eabase, float& abs_part, float& err) {
  i32x4 ex;
  asm volatile("ds_read_b128 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(ex) : "v"(eabase) : "memory");
  float part = 0.0f;
  abs_part = 0.0f;
  err = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    if ((uint32_t)b < nlive) {
      u32x4 a[4], xs[2];
      lds_read_group_block(iabase + 4096u * b, xabase + 32u * b, a, xs);
      float e;
      const float v = block_dot_tok<QB>(st, b, a, xs, ex[b], e);
      const bool fast = ex[b] != kBadBlock;
      const float c = fast ? v : 0.0f;
      part += c;
      abs_part += fabsf(c);
      err += fast ? e : 0.0f;
    }
  }
  return part;
}

// tok_group_stage with block_dot_tok_f64: the sum in f64, with abs_part and
// err (the bound on its rounding) as there.  Not inlined, and reading the
// stage again from its LDS buffer (ta: the lane's addresses there), so that
// its registers are taken on this rare path only.
struct StageF64 {
  double part;
  float abs_part, err;
};
template <int QB>
__device__ __noinline__ StageF64 tok_group_stage_f64(TokAddr ta, uint32_t nlive, uint32_t iabase,
                                                     uint32_t xabase, uint32_t eabase) {
  TokStage<QB> st;
  lds_read_weights_tok<QB>(ta, st);
  float abs_part, err;
  i32x4 ex;
  asm volatile("ds_read_b128 %0, %1\ns_waitcnt lgkmcnt(0)" : "=&v"(ex) : "v"(eabase) : "memory");
  double part = 0.0;
  abs_part = 0.0f;
  err = 0.0f;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    if ((uint32_t)b < nlive) {
      u32x4 a[4], xs[2];
      lds_read_group_block(iabase + 4096u * b, xabase + 32u * b, a, xs);
      float e;
      const double v = block_dot_tok_f64<QB>(st, b, a, xs, ex[b], e);
      const bool fast = ex[b] != kBadBlock;
      const double c = fast ? v : 0.0;
      part += c;
      abs_part += (float)fabs(c);
      err += fast ? e : 0.0f;
    }
  }
  return StageF64{part, abs_part, err};
}

// Side elements of a stage for the four vectors of one group (lane group r
// accumulates vector r of the group, row n).  list0 / cnt0: side lists and
// counts of the group's first vector at the stage's first block; the other
// vectors follow at side_stride).  For an entry (i, x_i) of
// vector r's block b, the lanes of group (i & 31) / 8 hold the qs byte of
// element i for their rows (slice (i / 32) / 2 of the block; Q5_K: and the
// qh byte of element i % 32 in their qh slice qh); lane group r takes w_i
// from them and adds w_i x_i.
template <int B, int QB>
__device__ __forceinline__ float tok_side_block(u32x4 h, u32x2 s0, u32x2 s1, u32x2 s2, u32x2 s3,
                                                u32x2 qh, uint32_t list, uint32_t counts,
                                                uint32_t r, uint32_t lane, float part) {
  const uint32_t grp = lane >> 4, n = lane & 15u;
  uint32_t c = (counts >> (8 * B)) & 0xffu;
  if (c == kSideRounded) c = 0u;
  for (uint32_t k = 0; k < c; ++k) {
    const u32x2 ent = lds_read_b64(list + kSideBytes * B + kSideEntryBytes * k);
    const uint32_t i = ent[0];  // the same in every lane
    const float xi = __uint_as_float(ent[1]);
    const uint32_t u = i >> 5, l = i & 31u, j = u >> 1;
    const u32x2 sl = j == 0u ? s0 : j == 1u ? s1 : j == 2u ? s2 : s3;
    const uint32_t byte = (((l & 4u) ? sl[1] : sl[0]) >> (8u * (l & 3u))) & 0xffu;
    uint32_t qv = (byte >> (4u * (u & 1u))) & 0x0fu;
    if constexpr (QB == 5) {
      const uint32_t hb = (((l & 4u) ? qh[1] : qh[0]) >> (8u * (l & 3u))) & 0xffu;
      qv |= ((hb >> u) & 1u) << 4;
    }
    const float wv = k4_weight(h, u, qv);
    const float wr = __int_as_float(
        __builtin_amdgcn_ds_bpermute((int)(4u * (16u * (l >> 3) + n)), __float_as_int(wv)));
    if (grp == r) part = fmaf(wr, xi, part);
  }
  return part;
}
// Largest |w| of a Q4_K (QMAX 15) or Q5_K (QMAX 31) block (all eight units)
// from its header.
template <int QMAX>
__device__ __forceinline__ float k4_block_bound(const u32x4& h) {
  const uint32_t sc03 = h[1] & 0x3f3f3f3fu;
  const uint32_t mn03 = h[2] & 0x3f3f3f3fu;
  const uint32_t sc47 = (h[3] & 0x0f0f0f0fu) | ((h[1] >> 2) & 0x30303030u);
  const uint32_t mn47 = ((h[3] >> 4) & 0x0f0f0f0fu) | ((h[2] >> 2) & 0x30303030u);
  const float ad = fabsf(half_bits_to_float(h[0] & 0xffffu));
  const float am = fabsf(half_bits_to_float(h[0] >> 16));
  float mx = 0.0f;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const uint32_t sc = ((u < 4 ? sc03 : sc47) >> (8 * (u & 3))) & 0xffu;
    const uint32_t mn = ((u < 4 ? mn03 : mn47) >> (8 * (u & 3))) & 0xffu;
    mx = fmaxf(mx, fmaf(ad, (float)((uint32_t)QMAX * sc), am * (float)mn));
  }
  return mx;
}

// Listed side elements of a stage for the four vectors of one group: lane
// (r, n) gets vector r's sum of w_i x_i over them for row n.  list0 / cnt0:
// side areas and counts of the group's first vector at the stage's first
// block (the other vectors at side_stride); `mine`: the lane's
// vector's counts.
template <int QB>
__device__ __forceinline__ float tok_listed(const TokStage<QB>& st, uint32_t list0, uint32_t mine,
                                            uint32_t side_stride, uint32_t lane) {
  const u32x4(&h)[4] = st.h;
  const u32x2(&q)[16] = st.q;
  auto qh = [&](int b) { return QB == 5 ? st.qh[QB == 5 ? b : 0] : u32x2{0u, 0u}; };
  float part = 0.0f;
  if (__builtin_amdgcn_ballot_w64((mine & ~(rounded_mask(mine) * 0xffu)) != 0u) == 0u)
    return part;
#pragma unroll 1
  for (uint32_t r = 0; r < 4u; ++r) {
    const uint32_t counts = __builtin_amdgcn_readlane(mine, 16 * r);
    if (counts == 0u) continue;
    const uint32_t list = list0 + r * side_stride;
    part = tok_side_block<0, QB>(h[0], q[0], q[1], q[2], q[3], qh(0), list, counts, r, lane,
                                 part);
    part = tok_side_block<1, QB>(h[1], q[4], q[5], q[6], q[7], qh(1), list, counts, r, lane,
                                 part);
    part = tok_side_block<2, QB>(h[2], q[8], q[9], q[10], q[11], qh(2), list, counts, r, lane,
                                 part);
    part = tok_side_block<3, QB>(h[3], q[12], q[13], q[14], q[15], qh(3), list, counts, r, lane,
                                 part);
  }
  return part;
}

// The lane's (vector r of the group, row n) error bound from its vector's
// rounded blocks of the stage: the largest |w| of each such block (from its
// header in h) times the block's error sum.
template <int QB>
__device__ __forceinline__ float tok_rounded_bound(uint32_t mine, uint32_t mylist,
                                                   const u32x4 (&h)[4]) {
  const uint32_t rmask = rounded_mask(mine);
  float err = 0.0f;
  if (__builtin_amdgcn_ballot_w64(rmask != 0u) == 0u) return err;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    if ((rmask >> b) & 1u)
      err = fmaf(k4_block_bound<QB == 5 ? 31 : 15>(h[b]), rounded_err_all(mylist + kSideBytes * b),
                 err);
  return err;
}

template <int WAVES, int NG, int QB>
__global__ __launch_bounds__(WAVES * 64) void q4k_tokens_mfma(const uint8_t* __restrict__ w,
                                                              const float* __restrict__ x,
                                                              float* __restrict__ y, uint32_t rows,
                                                              uint32_t nb, uint32_t ntok,
                                                              float* __restrict__ part_out,
                                                              TokArgs ta) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  constexpr uint32_t kPieces = block_pieces(QB);
  constexpr uint32_t kStage = stage_bytes(QB);
  constexpr uint32_t kBytes = QB == 5 ? kQ5Bytes : kQ4Bytes;
  const uint32_t wave = uniform(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t grp = lane >> 4, n = lane & 15u;
  const uint32_t row_bytes = nb * kBytes;
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + 3u) / 4u;
  const uint32_t sbase = (uint32_t)(uintptr_t)smem;
  uint8_t* const wstage = smem + wave * kStage;
  const bool sliced = ta.slices > 1u;
  const uint32_t ng = (ntok + 3u) / 4u;  // groups that hold vectors (<= NG)

  // this workgroup's slice k (stages [s0, s0 + spt)) and its tiles tg,
  // tg + GS, ...
  const FastDiv by_gps{ta.groups_per_slice, ta.m_gps};
  const uint32_t k = quo(blockIdx.x, by_gps);
  const uint32_t tg = blockIdx.x - k * ta.groups_per_slice;
  const uint32_t tstep = ta.groups_per_slice;
  const uint32_t s0 = sliced ? k : 0u, spt = sliced ? 1u : nstages;
  const uint32_t blk0 = 4u * s0, nbl = min(4u * spt, nb - blk0);
  const Layout L = tok_layout<QB>(WAVES, nbl, NG, ta.slots);
  const uint32_t ntw = tg < ntiles ? quo(ntiles - 1u - tg, by_gps) + 1u : 0u;
  const uint32_t npairs = ntw * spt;
  const FastDiv by_parts{spt, sliced ? 0u : ta.m_parts};

  // 1. the vectors' blocks of the range into the image area
  copy_x_group<WAVES>(smem, L.img, x, nb, blk0, nbl, ng, ntok, wave, lane);

  // 2. this wave's pairs p = wave, wave + WAVES, ...: local tile p / spt,
  //    stage s0 + p % spt; the first stage's copy goes out now
  const uint32_t my_pairs = wave < npairs ? (npairs - 1u - wave) / WAVES + 1u : 0u;
  const uint32_t voff = n * row_bytes + 16u * grp;
  auto pair_of = [&](uint32_t p) {
    Pair pr;
    const uint32_t i = quo(p, by_parts);
    pr.tile = tg + i * tstep;
    pr.r = s0 + (p - i * spt);
    pr.lt = i;
    pr.lo = 0u;
    pr.hi = spt;
    return pr;
  };
  auto issue = [&](const Pair& pr) {
    const uint32_t row0 = pr.tile * 16u;
    const uint32_t nrows = min(16u, rows - row0);
    const uint8_t* sb = w + (size_t)row0 * row_bytes + 4u * kBytes * pr.r;
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(sb), 0, (int)(nrows * row_bytes - 4u * kBytes * pr.r), kBufferWord3);
#pragma unroll
    for (int i = 0; i < (int)kPieces; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(wstage + 1024 * i), 16,
                                                voff + 64u * i, 0, 0, 0);
  };
  Pair pr_next = pair_of(wave);

  // 3. ring slots and the builders' count, set before any wave goes on (the
  //    waves start together, so this barrier costs little); every wave
  //    issues its first copy, and the waves that copied x blocks (a wave
  //    converts exactly the blocks it copied) build the group images once
  //    they have landed and count themselves done.  A wave reads images only
  //    once every builder has (wait_images), so no barrier makes a wave
  //    whose stage has landed wait for the waves whose copies the memory
  //    queue still holds back.  The first round of waves issues before the
  //    barrier (the empty queue takes their copies at once), the rest after.
  const bool first_round = wave < 4u;
  if (first_round && my_pairs > 0u) issue(pr_next);
  init_slots<WAVES>(sbase, L, ta.slots);
  lds_wait();
  __builtin_amdgcn_s_barrier();
  if (!first_round && my_pairs > 0u) issue(pr_next);
  const uint32_t builders = min((uint32_t)WAVES, ng * nbl);
  if (wave < builders) {
    if (my_pairs > 0u)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kPieces));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    build_group_images<WAVES, NG == 1>(sbase, L, nbl, ng, wave, lane);
    lds_wait();
    if (lane == 0u) (void)lds_add_rtn(sbase + L.ready, 1u);
  }

  // 4. the wave's pairs: lane (grp, n) accumulates, for each group g, vector
  //    4 g + grp, row n
  //    (the lane's 8-byte slices: qs bytes 32 j + 8 grp .. + 7 of unit pair j
  //    and, Q5_K, qh bytes 8 grp .. + 7)
  TokAddr sa;
  sa.hb0 = sbase + wave * kStage + 16u * n;
  sa.qhb0 = sa.hb0 + 256u * (1u + (grp >> 1)) + 8u * (grp & 1u);
  sa.qb0 = QB == 5 ? sa.qhb0 + 512u : sa.qhb0;
  uint32_t fail = 0u;  // a bounded wait that gave up (kDevErr*)
  for (uint32_t j = 0; j < my_pairs; ++j) {
    const Pair pr = pr_next;
    const uint32_t s = pr.r, sl = s - s0;  // stage, and its place in the image range
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    TokStage<QB> st;
    lds_read_weights_tok<QB>(sa, st);
    // the stage is in registers: the buffer takes the next stage's copy (the
    // exact path reads its blocks from memory), issued once the stage's
    // arithmetic is done: while the memory queue is full, issuing a copy
    // holds the wave
    auto issue_next = [&]() {
      if (j + 1u < my_pairs) {
        pr_next = pair_of(wave + (j + 1u) * WAVES);
        issue(pr_next);
      }
    };
    if (j == 0u) wait_images(sbase, L, builders, fail);
    const uint32_t nlive = min(4u, nb - 4u * s);
    bool any_bad = false;  // a block on the exact path
    // the lane's vector's side counts of each group, kept for the groups'
    // passes
    uint32_t counts[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) counts[g] = 0u;
    for (uint32_t g = 0; g < ng; ++g) {
      i32x4 ex;
      uint32_t cw;
      asm volatile(
          "ds_read_b128 %0, %2\n"
          "ds_read_b32 %1, %2 offset:512\n"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(ex), "=&v"(cw)
          : "v"(sbase + L.expo + (4u * g + grp) * L.expo_stride + 16u * sl)
          : "memory");
      cw = live_counts(cw, nlive);
#pragma unroll
      for (int gg = 0; gg < NG; ++gg)
        if ((uint32_t)gg == g) counts[gg] = cw;
      bool bad = false;
#pragma unroll
      for (int b = 0; b < 4; ++b) bad |= (uint32_t)b < nlive && ex[b] == kBadBlock;
      any_bad |= __builtin_amdgcn_ballot_w64(bad) != 0u;
    }
    float part[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) part[g] = 0.0f;
    uint32_t redo = 0u;  // bit g: the lane recomputes group g's stage exactly
    float rbs[NG];  // (two or four groups: each group's rounded-block bound)
    uint32_t redo_out = 0u;  // (K slices: bit g, tok_reduce recomputes it)
    // (groups one after another: unrolled, their registers would add up)
#pragma unroll 1
    for (uint32_t g = 0; g < (NG == 1 ? 1u : ng); ++g) {
      const uint32_t v = 4u * g + grp;
      uint32_t mine = counts[0];
#pragma unroll
      for (int gg = 1; gg < NG; ++gg)
        if ((uint32_t)gg == g) mine = counts[gg];
      const bool any = __builtin_amdgcn_ballot_w64(mine != 0u) != 0u;
      const uint32_t list0 =
          sbase + L.expo + 4u * g * L.expo_stride + L.side_off + 4u * kSideBytes * sl;
      // (listed side elements: one group only; with more, side elements make
      // rounded blocks)
      float side = 0.0f;
      if constexpr (NG == 1)
        side = any ? tok_listed<QB>(st, list0, mine, L.expo_stride, lane) : 0.0f;
      float abs_pg, err;
      const uint32_t iabase = sbase + L.img + 4096u * (g * nbl + 4u * sl) + 16u * lane;
      const uint32_t xabase = sbase + L.xsum + v * L.xsum_stride + 128u * sl;
      const uint32_t eabase = sbase + L.expo + v * L.expo_stride + 16u * sl;
      float pg = side + tok_group_stage<QB>(st, nlive, iabase, xabase, eabase, abs_pg, err);
      // the stage check of the lane's (vector, row): the fast path's rounding
      // plus its rounded blocks against kStageTol of sum |partial|
      const float rb = any ? tok_rounded_bound<QB>(mine, list0 + grp * L.expo_stride, st.h) : 0.0f;
      err += rb;
      const bool failed = !(err * 1.01f <= kStageTol * (abs_pg + fabsf(side) - err));
      // One group (M <= 4): a lane that fails tries the stage again with the
      // digit sums combined in f64 (a bound about eight times tighter; the
      // stage is still in its LDS buffer, the images beside it) before it is
      // left to the exact path, whose reads of weights from memory cost a
      // launch 2.5 us of tail at about one failing lane in 2e4: M = 4 20.5 ->
      // 18.6 us.  Made here, the call costs the two- and four-group kernels
      // spills in their main loop (M = 8 31 -> 45 us); they make it after the
      // groups' loop (below).
      if (NG == 1 && __builtin_amdgcn_ballot_w64(failed) != 0u) {
        const StageF64 sp = tok_group_stage_f64<QB>(sa, nlive, iabase, xabase, eabase);
        const float err_p = sp.err + rb;
        if (failed) {
          if (err_p * 1.01f <= kStageTol * (sp.abs_part + fabsf(side) - err_p))
            pg = side + (float)sp.part;
          else
            redo |= 1u << g;
        }
      } else if (NG > 1 && failed) {
        redo |= 1u << g;
      }
#pragma unroll
      for (int gg = 0; gg < NG; ++gg)
        if ((uint32_t)gg == g) {
          part[gg] = pg;
          rbs[gg] = rb;
        }
    }
    // Two or four groups: the lanes that failed try their groups' stages
    // again in f64 once the groups' loop is done, one group at a time; what
    // still fails goes to the exact path.  At M = 8 on Q4_K 17408x5120 about
    // one stage lane in 2e4 fails the f32 check: left to tok_reduce, they
    // gave 35 of its 544 workgroups an exact recompute (a second trip to
    // memory) and the pass its tail.  Tried here, none is left: M = 8 / 16
    // 28.5 / 42.6 -> 27.1 / 41.6 us, Q5_K 5120x5120 16.7 / 27.1 -> 15.3 /
    // 25.1 us.
    if constexpr (NG > 1) {
      if (__builtin_amdgcn_ballot_w64(redo != 0u) != 0u) {
#pragma unroll 1
        for (uint32_t g = 0; g < ng; ++g) {
          if (__builtin_amdgcn_ballot_w64((redo >> g) & 1u) == 0u) continue;
          const uint32_t v = 4u * g + grp;
          const StageF64 sp = tok_group_stage_f64<QB>(
              sa, nlive, sbase + L.img + 4096u * (g * nbl + 4u * sl) + 16u * lane,
              sbase + L.xsum + v * L.xsum_stride + 128u * sl,
              sbase + L.expo + v * L.expo_stride + 16u * sl);
          float rb = rbs[0];
#pragma unroll
          for (int gg = 1; gg < NG; ++gg)
            if ((uint32_t)gg == g) rb = rbs[gg];
          const float err_p = sp.err + rb;
          if (((redo >> g) & 1u) && err_p * 1.01f <= kStageTol * (sp.abs_part - err_p)) {
            redo &= ~(1u << g);
#pragma unroll
            for (int gg = 0; gg < NG; ++gg)
              if ((uint32_t)gg == g) part[gg] = (float)sp.part;
          }
        }
      }
    }
    // a K-sliced launch leaves the stages of lanes that failed the check to
    // tok_reduce (kPartRedo below); the others take the exact path here
    if (sliced) redo_out = redo;
    const uint32_t redo_here = sliced ? 0u : redo;
    if (any_bad || __builtin_amdgcn_ballot_w64(redo_here != 0u) != 0u) {
      // the rare exact path: one loop over (group, block), weights read from
      // memory, the rest addressed in LDS (no register array indexed at run
      // time)
      const uint32_t row0 = pr.tile * 16u;
      const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(w + (size_t)row0 * row_bytes), 0,
          (int)(min(16u, rows - row0) * row_bytes), kBufferWord3);
#pragma unroll 1
      for (uint32_t g = 0; g < ng; ++g) {
        const uint32_t v = 4u * g + grp;
        const float* const xv = x + (size_t)min(v, ntok - 1u) * nb * kBlockElems;
        const bool whole = (redo_here >> g) & 1u;
        float e = 0.0f;
#pragma unroll 1
        for (uint32_t b = 0; b < nlive; ++b) {
          const uint32_t eb = lds_read_b32(sbase + L.expo + v * L.expo_stride + 4u * (4u * sl + b));
          if ((int)eb == kBadBlock || whole)
            e += block_exact_row<QB>(wr, n * row_bytes + kBytes * (4u * s + b),
                                 xv + kBlockElems * (4u * s + b));
        }
#pragma unroll
        for (int gg = 0; gg < NG; ++gg)
          if ((uint32_t)gg == g) part[gg] = (whole ? 0.0f : part[gg]) + e;
      }
    }
    issue_next();
    if (!sliced) {
      hand_off_lane_tokens(sbase, L, FastDiv{ta.slots, ta.m_slots}, pr, nstages, part[0], lane,
                           rows, ntok, y, fail);
      continue;
    }
    // the stage's partial sums of the tile's rows, for tok_reduce
    const uint32_t row = pr.tile * 16u + n;
    if (row < rows) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const uint32_t v = 4u * g + grp;
        if (v < ntok)
          part_out[((size_t)s * 4u * NG + v) * rows + row] =
              ((redo_out >> g) & 1u) ? __uint_as_float(kPartRedo) : part[g];
      }
    }
  }
  if (fail != 0u) report_device_error(ta.wsp, fail);
}

// Slice count of a launch: one per stage when the stages' partial sums of
// nv vectors fit the workspace's scratch and every slice still has a
// workgroup, else 1 (whole rows).
inline uint32_t tok_slices(uint32_t rows, uint32_t nstages, uint32_t nv, size_t scratch_bytes) {
  const uint32_t cus = (uint32_t)cu_count();
  if (nstages < 2u || nstages > cus) return 1u;
  if ((size_t)nstages * nv * rows * sizeof(float) > scratch_bytes) return 1u;
  return nstages;
}

// ntok <= 4 NG vectors in one pass; false when the shape does not fit this
// kernel (K slices need room in the scratch when NG > 1).
template <int W, int NG, int QB = 4>
bool launch_tokens_td(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                      uint32_t ntok, const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + 3u) / 4u;
  TokArgs ta{};
  uint32_t grid, lds;
  ta.slices = tok_slices(rows, nstages, 4u * NG, ws.scratch_bytes);
  if (ta.slices > 1u) {
    ta.groups_per_slice = min((uint32_t)cu_count() / ta.slices, ntiles);
    ta.slots = 1u;
    grid = ta.groups_per_slice * ta.slices;
    lds = tok_layout<QB>(W, min(4u, nb), NG, 1u).total;
  } else {
    if (NG > 1) return false;  // whole rows: one group's images already fill the LDS
    ta.groups_per_slice = grid = min(ntiles, (uint32_t)cu_count());
    const uint32_t tiles_per_group = (ntiles + grid - 1u) / grid;
    ta.slots = ring_slots(W, 1, tiles_per_group, nstages);
    ta.m_parts = div_magic(nstages);
    lds = tok_layout<QB>(W, nb, NG, ta.slots).total;
    // pair indices below tiles_per_group * nstages, divided by nstages
    if ((uint64_t)tiles_per_group * nstages * nstages >= (1ull << 32)) return false;
  }
  ta.m_gps = div_magic(ta.groups_per_slice);
  ta.m_slots = div_magic(ta.slots);
  ta.wsp = ws.ptr;
  // block and tile indices divided by GS
  if ((uint64_t)(grid + ntiles) * ta.groups_per_slice >= (1ull << 32)) return false;
  if (lds > kLdsBytes) return false;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&q4k_tokens_mfma<W, NG, QB>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q4k_tokens_mfma<W, NG, QB>), dim3(grid), dim3(W * 64), lds, s, w, x, y, rows,
                     nb, ntok, ws.scratch, ta);
  *err = hipGetLastError();
  if (*err == hipSuccess && ta.slices > 1u) {
    launch_tok_reduce<QB == 5 ? kTypeQ5K : kTypeQ4K>(ws.scratch, y, rows, nstages, 4u * NG, ntok,
                                                     w, x, nb, 4u, s);
    *err = hipGetLastError();
  }
  return true;
}

// 3..16 vectors in one launch (with its reduce): the group count and wave
// count that fit.
template <int QB>
bool launch_tokens_groups(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                          uint32_t ntok, const Workspace& ws, hipStream_t s, hipError_t* err) {
  if (ntok <= 4u) {
    if constexpr (QB == 4) {
      if (launch_tokens_td<12, 1, QB>(w, x, y, rows, nb, ntok, ws, s, err)) return true;
    }
    return launch_tokens_td<8, 1, QB>(w, x, y, rows, nb, ntok, ws, s, err) ||
           launch_tokens_td<4, 1, QB>(w, x, y, rows, nb, ntok, ws, s, err);
  }
  // (the weights' decoded operands stay in registers across the groups: two
  // waves per SIMD)
  if (ntok <= 8u) return launch_tokens_td<8, 2, QB>(w, x, y, rows, nb, ntok, ws, s, err);
  return launch_tokens_td<8, 4, QB>(w, x, y, rows, nb, ntok, ws, s, err) ||
         launch_tokens_td<6, 4, QB>(w, x, y, rows, nb, ntok, ws, s, err);
}

template <int W, int D, int M, int NT = 1, int QB = 4, bool G = false, int SB = 4,
          bool LN = false>
bool launch_wd(const uint8_t* w, const uint8_t* w2, const float* x, float* y, uint32_t rows,
               uint32_t nb, const Workspace& ws, hipStream_t s, hipError_t* err,
               const GroupArgs& ga = GroupArgs{}) {
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t tstages = (nb + SB - 1u) / SB * M;
  // several vectors: whole tiles only
  const LaunchShape ls = launch_shape(ntiles, tstages, W, NT == 1 ? ws.bytes : 0u, M);
  const uint32_t grid = ls.groups;
  const uint32_t slots = ring_slots(W, D, ls.tiles_per_group, tstages);
  const uint32_t lds = layout(W, D, nb, slots, M, NT, QB, SB, LN).total;
  SchedArgs sa;
  if (lds > kLdsBytes || !make_sched_args(ntiles, tstages, slots, ls, &sa)) return false;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&q4k_matvec_mfma<W, D, M, NT, QB, G, false, SB, LN>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q4k_matvec_mfma<W, D, M, NT, QB, G, false, SB, LN>), dim3(grid),
                     dim3(W * 64), lds, s, w, w2, x, y, rows, nb, ws.ptr, sa, ga, SliceArgs{});
  *err = hipGetLastError();
  return true;
}

// Whether a Q4_K launch of whole rows can take full-line copies: four-block
// stages that fill every row, rows of 144 nb bytes with nb = 4 mod 8 (64
// bytes past a whole number of lines) and 128-byte aligned matrices, so that
// every tile starts on a line.
bool lines_fit(uint32_t nb, const uint8_t* w, const uint8_t* w2 = nullptr) {
  static const int env = env_int("SI_HIP_Q4K_LINES", 1);
  auto aligned = [](const uint8_t* p) { return ((uintptr_t)p & 127u) == 0u; };
  return env != 0 && nb % 8u == 4u && aligned(w) && (w2 == nullptr || aligned(w2));
}

// A K-sliced launch of one vector in S slices (false when the shape or the
// LDS does not fit).  The slice's blocks, not the row's, bound the LDS
// metadata, so rows longer than the unsliced kernels take run here.
template <int W, int D, int QB, int SB = 4>
bool launch_sliced(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                   uint32_t S, const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t ntiles = (rows + 15u) / 16u;
  const uint32_t nstages = (nb + SB - 1u) / SB;
  if (rows == 0u || nb == 0u || (uint64_t)nb * block_bytes(QB) * 16u > 0x7fffffffu) return false;
  SliceShape sh;
  if (!slice_shape(ntiles, nstages, S, (uint32_t)cu_count(), ws.bytes, &sh)) return false;
  if (SB * sh.ns_max > kMaxMetaBlocks) return false;
  const uint32_t slots = ring_slots(W, D, sh.tiles_per_group, sh.ns_max);
  const uint32_t lds = layout(W, D, SB * sh.ns_max, slots, 1u, 1u, QB, SB).total;
  if (lds > kLdsBytes || slots > 0xffu || sh.groups > 0xffffu) return false;
  SchedArgs sa{};
  sa.packed = (sh.groups << 16) | slots;
  sa.m_slots = div_magic(slots);
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&q4k_matvec_mfma<W, D, 1, 1, QB, false, true, SB>),
      hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsBytes);
  if (attr != hipSuccess) {
    *err = attr;
    return true;
  }
  hipLaunchKernelGGL((q4k_matvec_mfma<W, D, 1, 1, QB, false, true, SB>), dim3(sh.groups),
                     dim3(W * 64), lds, s, w, nullptr, x, y, rows, nb, ws.ptr, sa, GroupArgs{},
                     sh.args);
  *err = hipGetLastError();
  return true;
}

// Slices for a one-vector Q4_K / Q5_K launch, or 0.  The same rule as the
// Q6_K kernel's (q6_slices), measured on this kernel (MI355X, us):
//   type  rows x cols    unsliced  S = 2   S = 4   S = 8
//   Q4_K  5120 x 17408     18.3     18.3    16.5    21.5
//   Q4_K  2048 x 16384     12.4     10.0     9.0    10.2
//   Q4_K  640 x 17408      11.5      9.3     8.0     8.5
//   Q4_K  8192 x 28672    140.0     38.1    34.9    41.1   (unsliced: 4 waves)
//   Q4_K  2560 x 34816     75.7     22.8    18.8    18.2   (unsliced: generic kernel)
//   Q4_K  2560 x 9728       8.6      9.1     8.6     9.7
//   Q4_K  17408 x 5120     13.6     17.7    22.7
//   Q4_K  5120 x 5120       7.7      8.1     8.8
//   Q4_K  8192 x 8192      11.5              15.6
//   Q4_K  12288 x 8192     15.0              18.5
//   Q4_K  4096 x 8192       8.9               9.4
//   Q4_K  4096 x 12288     10.3              10.5            (unsliced: 8 waves)
//   Q5_K  5120 x 17408     25.6     23.9    22.1    27.0
//   Q5_K  5120 x 5120       9.2     11.2    11.7
// So: rows of fewer than 8 stages (K < 8192) stay whole; four slices when
// the unsliced launch's busiest workgroup has at most two rounds of pairs
// (24) and slicing takes some of them (a tie keeps the whole rows) or the
// rows are long (64 blocks or more); with more pairs, only rows whose
// images leave room for fewer than eight waves (or exceed the LDS
// metadata), in four slices, else two, when that adds no pairs.  Rows
// longer than the unsliced kernels take must slice.
// The (tile, stage) pairs of an unsliced launch's busiest workgroup, on
// launch_shape's grid at the given wave count.
uint64_t busiest_pairs(uint32_t ntiles, uint32_t tparts, uint32_t waves, size_t ws_bytes) {
  const LaunchShape ls = launch_shape(ntiles, tparts, waves, ws_bytes, 1u);
  const uint64_t g = ls.groups, q = ntiles / g, lp = (ntiles - q * g) * (uint64_t)tparts;
  return ls.split ? q * tparts + (lp + g - 1u) / g : (ntiles + g - 1u) / g * tparts;
}

// Whether an unsliced one-vector launch of W waves and SB-block stages fits
// the LDS.
bool unsliced_fits(uint32_t ntiles, uint32_t nb, uint32_t waves, int qb, int sb,
                   size_t ws_bytes) {
  const uint32_t tparts = (nb + sb - 1u) / sb;
  const LaunchShape ls = launch_shape(ntiles, tparts, waves, ws_bytes, 1u);
  const uint32_t slots = ring_slots(waves, 1u, ls.tiles_per_group, tparts);
  return layout(waves, 1u, nb, slots, 1u, 1u, qb, sb).total <= kLdsBytes;
}

struct SliceChoice {
  uint32_t slices = 0;   // 0: unsliced
  uint64_t most0 = 0;    // busiest unsliced workgroup's pairs (0: not weighed)
  uint64_t most_s = 0;   // busiest sliced workgroup's pairs at `slices`
  bool forced = false;   // SI_HIP_Q4K_SLICES fixed `slices`
};

SliceChoice q4_slices(uint32_t ntiles, uint32_t nb, size_t ws_bytes, int qb) {
  SliceChoice c;
  static const int env = env_int("SI_HIP_Q4K_SLICES", -1);
  if (env >= 0) {
    c.slices = (uint32_t)env;
    c.forced = true;
    return c;
  }
  const uint32_t nst = (nb + 3u) / 4u;
  if (nst < 8u) return c;
  const uint64_t cus = (uint64_t)cu_count();
  auto most = [&](uint32_t S) {  // the busiest sliced workgroup's pairs
    const uint64_t gs = std::min<uint64_t>(ntiles, cus / S);
    return (ntiles + gs - 1u) / gs * ((nst + S - 1u) / S);
  };
  if (nb > kMaxMetaBlocks) {
    // rows longer than the unsliced kernels take must slice: the fewest
    // slices (from four) whose images leave the stage buffers of 12 waves
    // (Q4_K, 32 blocks) or 8 (Q5_K, 64 blocks) room in the LDS
    const uint32_t cap = qb == 5 ? 16u : 8u;  // stages per slice
    uint32_t S = 4u;
    while (S < 64u && S < cus && (nst + S - 1u) / S > cap) S *= 2u;
    c.slices = S;
    return c;
  }
  c.most0 = busiest_pairs(ntiles, nst, qb == 5 ? 8u : 12u, ws_bytes);
  auto pick = [&](uint32_t S) {
    c.slices = S;
    c.most_s = most(S);
    return c;
  };
  if (c.most0 <= 24u) return most(4u) < c.most0 || nb >= 64u ? pick(4u) : c;
  if (layout(8u, 1u, nb, 2u, 1u, 1u, qb).total <= kLdsBytes) return c;
  for (uint32_t S : {4u, 2u})
    if (most(S) <= c.most0) return pick(S);
  return c;
}

// Whether one Q4_K / Q5_K vector runs as two-block stages (12 waves,
// unsliced) rather than the slices of `sc` or four-block stages.  A stage of
// two blocks halves each pair, so more waves share a short launch; it costs
// more per block (twice the pairs, hand-offs and waits).  Measured on MI355X
// (us; the four-block kernel unsliced at 12 waves, or at 8 where 12 do not
// fit):
//   type  rows x cols    4-block  sliced  2-block
//   Q4_K  4096 x 4096       5.6      -       5.2
//   Q4_K  8192 x 5120       8.0      -       7.5
//   Q4_K  5120 x 5120       7.6      -       7.1
//   Q4_K  1024 x 5120       6.1      -       5.6
//   Q4_K  4096 x 8192       8.9     9.4      8.1
//   Q4_K  8192 x 6144       8.6      -       9.1   (12 pairs per workgroup)
//   Q4_K  8192 x 8192      11.5    15.6     12.4   (16)
//   Q4_K  17408 x 5120     13.8      -      14.8   (22)
//   Q4_K  4096 x 14336     11.8    13.6     11.4   (12 waves do not fit)
//   Q4_K  2048 x 11008      -       8.4      8.9
//   Q4_K  1024 x 17408     11.2     8.1     10.7
//   Q5_K  5120 x 5120       9.1      -       7.9
//   Q5_K  8192 x 8192      16.0    16.6     14.6
//   Q5_K  17408 x 5120     18.0      -      18.1
//   Q5_K  5120 x 17408     22.2    22.2     20.3
//   Q5_K  2560 x 17408      -      15.0     15.7
//   Q5_K  640 x 17408       -       8.7     11.4
//   Q5_K  1024 x 8192       -       7.9      8.3
// So Q4_K takes two-block stages when the four-block launch leaves waves
// idle (fewer pairs per workgroup than waves) and the two-block one needs at
// most two rounds, or when 12 waves of four-block stages do not fit (three
// rounds); Q5_K, whose four-block stages leave registers for only 8 waves,
// whenever 12 waves fit.  Slices stay where every unsliced workgroup would
// build the whole row's activation images for a small share of the work:
// at most a quarter as many tiles as CUs, rows of 64 blocks or more over
// fewer tiles than CUs, and rows past 32 blocks whose busiest workgroup the
// slices shorten.
bool two_block_stages(uint32_t ntiles, uint32_t nb, size_t ws_bytes, int qb,
                      const SliceChoice& sc) {
  constexpr uint32_t kWaves = 12u;
  if (sc.forced || !unsliced_fits(ntiles, nb, kWaves, qb, 2, ws_bytes)) return false;
  const uint32_t cus = (uint32_t)cu_count();
  if (sc.slices >= 2u && (ntiles <= cus / 4u || (nb >= 64u && ntiles < cus) ||
                          (nb > 32u && sc.most_s < sc.most0)))
    return false;
  if (qb == 5) return true;
  if (nb > 56u) return false;
  const uint64_t rounds2 = (busiest_pairs(ntiles, (nb + 1u) / 2u, kWaves, ws_bytes) + kWaves - 1u) /
                           kWaves;
  if (!unsliced_fits(ntiles, nb, kWaves, qb, 4, ws_bytes)) return rounds2 <= 3u;
  return rounds2 <= 2u && busiest_pairs(ntiles, (nb + 3u) / 4u, kWaves, ws_bytes) < kWaves;
}

// Whether the unsliced kernel of SB-block stages takes the shape (the
// offsets, pair counts and quotients its schedule forms).
bool shape_ok(uint32_t rows, uint32_t cols, uint32_t mats, int qb, uint32_t sb = 4u) {
  const uint32_t nb = cols / kBlockElems;
  const uint64_t pairs = (uint64_t)((rows + 15u) / 16u) * ((nb + sb - 1u) / sb) * mats;
  return rows != 0 && nb != 0 && nb <= kMaxMetaBlocks &&
         (uint64_t)nb * block_bytes(qb) * 16u <= 0x7fffffffu &&
         (uint64_t)nb * 1024u <= 0x7fffffffu && pairs <= 0xffffffffu &&
         quotients_fit((rows + 15u) / 16u, (nb + sb - 1u) / sb * mats);
}

// Whether a sliced launch takes two-block stages: when the busiest sliced
// workgroup of four-block stages has fewer pairs than 12 waves, so that
// waves would idle.  Measured on MI355X (us, S = 4, four- / two-block):
// Q4_K 1024 x 17408 7.62 / 7.17, 640 x 17408 7.27 / 6.99, 2048 x 16384 8.39 /
// 8.14, 1000 x 12800 7.07 / 6.69, 2048 x 11008 7.53 / 7.37; Q5_K 1024 x 17408
// 8.48 / 7.77, 2048 x 16384 9.40 / 8.85; with more pairs four-block stages
// win: Q4_K 2560 x 17408 9.94 / 11.95, 5120 x 17408 16.2 / 19.9.
// SI_HIP_Q4K_SLICE_SB (2 or 4) fixes the choice.
bool sliced_two_block(uint32_t ntiles, uint32_t nb, uint32_t S, size_t ws_bytes) {
  static const int env = env_int("SI_HIP_Q4K_SLICE_SB", 0);
  if (env == 2 || env == 4) return env == 2;
  SliceShape sh;
  if (!slice_shape(ntiles, (nb + 3u) / 4u, S, (uint32_t)cu_count(), ws_bytes, &sh)) return false;
  return (uint64_t)sh.tiles_per_group * sh.ns_max < 12u;
}

// Two-block stages or the sliced launch, when two_block_stages or q4_slices
// asks for one.
template <int QB>
bool try_sliced(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t cols,
                const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  if (rows == 0u || nb == 0u) return false;
  const uint32_t ntiles = (rows + 15u) / 16u;
  const SliceChoice sc = q4_slices(ntiles, nb, ws.bytes, QB);
  if (shape_ok(rows, cols, 1u, QB, 2u) && two_block_stages(ntiles, nb, ws.bytes, QB, sc) &&
      launch_wd<12, 1, 1, 1, QB, false, 2>(w, nullptr, x, y, rows, nb, ws, s, err))
    return true;
  const uint32_t S = sc.slices;
  if (S < 2u) return false;
  if (sliced_two_block(ntiles, nb, S, ws.bytes) &&
      launch_sliced<12, 1, QB, 2>(w, x, y, rows, nb, S, ws, s, err))
    return true;
  if constexpr (QB == 4) {  // (Q5_K's weight registers leave room for 8 waves)
    if (launch_sliced<12, 1, QB>(w, x, y, rows, nb, S, ws, s, err)) return true;
  }
  return launch_sliced<8, 1, QB>(w, x, y, rows, nb, S, ws, s, err) ||
         launch_sliced<4, 1, QB>(w, x, y, rows, nb, S, ws, s, err);
}

// NT activation vectors (batch-major x and y) in one pass over the weights.
template <int NT, int QB>
bool launch_tokens(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                   const Workspace& ws, hipStream_t s, hipError_t* err) {
  return launch_wd<8, 1, 1, NT, QB>(w, nullptr, x, y, rows, nb, ws, s, err) ||
         launch_wd<6, 1, 1, NT, QB>(w, nullptr, x, y, rows, nb, ws, s, err) ||
         launch_wd<4, 1, 1, NT, QB>(w, nullptr, x, y, rows, nb, ws, s, err);
}


// One vector, Q5_K in four-block stages (8 waves: their 20 weight pieces per
// wave leave too few registers for 12).
bool launch_q5k_one(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t nb,
                    const Workspace& ws, hipStream_t s, hipError_t* err) {
  static const int cfg = env_int("SI_HIP_Q5K_MFMA_CFG", 0);
  switch (cfg) {
    case 1: return launch_wd<8, 1, 1, 1, 5>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 2:
      return shape_ok(rows, nb * kBlockElems, 1u, 5, 2u) &&
             launch_wd<12, 1, 1, 1, 5, false, 2>(w, nullptr, x, y, rows, nb, ws, s, err);
    default: break;
  }
  return launch_wd<8, 1, 1, 1, 5>(w, nullptr, x, y, rows, nb, ws, s, err) ||
         launch_wd<4, 1, 1, 1, 5>(w, nullptr, x, y, rows, nb, ws, s, err);
}

// SI_HIP_TOKENS_TD=0 keeps the one-vector-per-MFMA kernel for batches
inline bool td_policy() {
  static const int v = env_int("SI_HIP_TOKENS_TD", 1);
  return v != 0;
}

// batch >= 2 vectors: three to sixteen in one pass of the vectors-in-rows
// kernel, two (or, under SI_HIP_TOKENS_TD=0, up to four) per pass of the
// one-vector-per-MFMA kernel
template <int QB>
bool matmul_passes(const uint8_t* w, const float* x, float* y, uint32_t rows, uint32_t cols,
                   uint32_t batch, const Workspace& ws, hipStream_t s, hipError_t* err) {
  const uint32_t nb = cols / kBlockElems;
  for (uint32_t b = 0; b < batch;) {
    const uint32_t nt = min(4u, batch - b);
    const float* xb = x + (size_t)b * cols;
    float* yb = y + (size_t)b * rows;
    bool ok;
    if (nt >= 2 && td_policy()) {
      // up to sixteen vectors share the matrix-core rows in one pass (two
      // go faster one vector per MFMA)
      const uint32_t ng = batch - b >= 3u ? min(16u, batch - b) : nt;
      if (ng >= 3u && launch_tokens_groups<QB>(w, xb, yb, rows, nb, ng, ws, s, err)) {
        if (*err != hipSuccess) return true;
        b += ng;
        continue;
      }
    }
    switch (nt) {
      case 4: ok = launch_tokens<4, QB>(w, xb, yb, rows, nb, ws, s, err); break;
      case 3: ok = launch_tokens<3, QB>(w, xb, yb, rows, nb, ws, s, err); break;
      case 2: ok = launch_tokens<2, QB>(w, xb, yb, rows, nb, ws, s, err); break;
      default:
        ok = QB == 5 ? launch_q5k_matvec_mfma(w, xb, yb, rows, cols, ws, s, err)
                     : launch_q4k_matvec_mfma(w, xb, yb, rows, cols, ws, s, err);
        break;
    }
    if (!ok) {
      if (b == 0) return false;
      *err = hipErrorInvalidValue;
      return true;
    }
    if (*err != hipSuccess) return true;
    b += nt;
  }
  return true;
}

}  // namespace

bool launch_q4k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err) {
  static const int cfg = env_int("SI_HIP_Q4K_MFMA_CFG", 0);
  if (cfg == 0 && try_sliced<4>(w, x, y, rows, cols, ws, s, err)) return true;
  if (!shape_ok(rows, cols, 1u, 4)) return false;
  const uint32_t nb = cols / kBlockElems;
  switch (cfg) {
    case 5:
      return shape_ok(rows, cols, 1u, 4, 2u) &&
             launch_wd<12, 1, 1, 1, 4, false, 2>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 1: return launch_wd<12, 1, 1>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 2: return launch_wd<8, 1, 1>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 3: return launch_wd<4, 3, 1>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 4: return launch_wd<5, 3, 1>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 6:
      return lines_fit(nb, w) &&
             launch_wd<6, 2, 1, 1, 4, false, 4, true>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 7:
      return lines_fit(nb, w) &&
             launch_wd<12, 1, 1, 1, 4, false, 4, true>(w, nullptr, x, y, rows, nb, ws, s, err);
    case 8:
      return lines_fit(nb, w) &&
             launch_wd<8, 1, 1, 1, 4, false, 4, true>(w, nullptr, x, y, rows, nb, ws, s, err);
    default: break;
  }
  // full-line copies where the shape allows them, measured on MI355X
  // (17408 x 5120, us, back to back over 8 resident copies): 12 waves 13.1,
  // 8 waves 13.5, 6 waves with two stages in flight 15.9 (the stage
  // arithmetic needs three waves per SIMD to hide its latency); the
  // half-line copies at 12 waves 13.6
  if (lines_fit(nb, w) &&
      launch_wd<12, 1, 1, 1, 4, false, 4, true>(w, nullptr, x, y, rows, nb, ws, s, err))
    return true;
  return launch_wd<12, 1, 1>(w, nullptr, x, y, rows, nb, ws, s, err) ||
         launch_wd<8, 1, 1>(w, nullptr, x, y, rows, nb, ws, s, err) ||
         launch_wd<4, 1, 1>(w, nullptr, x, y, rows, nb, ws, s, err);
}

static_assert(kMaxGroupWeights == kMaxGroup, "the C ABI's group limit is the kernels'");

bool launch_matvec_group(uint32_t type, const uint8_t* const* w, const uint32_t* rows,
                         uint32_t count, uint32_t cols, const float* x, float* y,
                         const Workspace& ws, hipStream_t s, hipError_t* err) {
  if (count < 2u || count > kMaxGroup) return false;
  GroupArgs ga{};
  for (uint32_t k = 0; k < kMaxGroup; ++k) ga.tile_end[k] = 0xffffffffu;
  uint64_t tiles = 0, total = 0;
  for (uint32_t k = 0; k < count; ++k) {
    if (rows[k] == 0u || (k + 1u < count && rows[k] % 16u != 0u)) return false;
    ga.w[k] = w[k];
    ga.rows[k] = rows[k];
    total += rows[k];
    tiles += (rows[k] + 15u) / 16u;
    if (total > 0xffffffffu) return false;
    ga.tile_end[k] = (uint32_t)tiles;
  }
  const uint32_t nb = cols / kBlockElems, trows = (uint32_t)total;
  // two-block stages where one matrix of the group's rows would take them
  static const int group_two_block = env_int("SI_HIP_GROUP_TWO_BLOCK", 1);
  if (group_two_block != 0 && (type == kTypeQ4K || type == kTypeQ5K) && shape_ok(trows, cols, 1u, type == kTypeQ4K ? 4 : 5, 2u) &&
      two_block_stages((uint32_t)tiles, nb, ws.bytes, type == kTypeQ4K ? 4 : 5, SliceChoice{})) {
    if (type == kTypeQ4K &&
        launch_wd<12, 1, 1, 1, 4, true, 2>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga))
      return true;
    if (type == kTypeQ5K &&
        launch_wd<12, 1, 1, 1, 5, true, 2>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga))
      return true;
  }
  switch (type) {
    case kTypeQ4K:
      return shape_ok(trows, cols, 1u, 4) &&
             (launch_wd<12, 1, 1, 1, 4, true>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga) ||
              launch_wd<8, 1, 1, 1, 4, true>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga));
    case kTypeQ5K:
      return shape_ok(trows, cols, 1u, 5) &&
             (launch_wd<8, 1, 1, 1, 5, true>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga) ||
              launch_wd<4, 1, 1, 1, 5, true>(w[0], nullptr, x, y, trows, nb, ws, s, err, ga));
    case kTypeQ6K:
      return launch_q6k_matvec_group(ga, trows, cols, x, y, ws, s, err);
    default:
      return false;
  }
}

bool launch_q5k_matvec_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, const Workspace& ws, hipStream_t s, hipError_t* err) {
  static const int cfg = env_int("SI_HIP_Q5K_MFMA_CFG", 0);
  if (cfg == 0 && try_sliced<5>(w, x, y, rows, cols, ws, s, err)) return true;
  if (!shape_ok(rows, cols, 1u, 5)) return false;
  return launch_q5k_one(w, x, y, rows, cols / kBlockElems, ws, s, err);
}

bool launch_q4k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err) {
  if (batch < 2 || !shape_ok(rows, cols, 1u, 4)) return false;
  return matmul_passes<4>(w, x, y, rows, cols, batch, ws, s, err);
}

bool launch_q5k_matmul_mfma(const uint8_t* w, const float* x, float* y, uint32_t rows,
                            uint32_t cols, uint32_t batch, const Workspace& ws, hipStream_t s,
                            hipError_t* err) {
  if (batch < 2 || !shape_ok(rows, cols, 1u, 5)) return false;
  return matmul_passes<5>(w, x, y, rows, cols, batch, ws, s, err);
}

bool launch_q4k_gate_up_mfma(const uint8_t* gate, const uint8_t* up, const float* x, float* h,
                             uint32_t rows, uint32_t cols, const Workspace& ws, hipStream_t s,
                             hipError_t* err) {
  if (!shape_ok(rows, cols, 2u, 4)) return false;
  const uint32_t nb = cols / kBlockElems;
  static const int cfg = env_int("SI_HIP_GATE_UP_MFMA_CFG", 0);
  switch (cfg) {
    case 1: return launch_wd<12, 1, 2>(gate, up, x, h, rows, nb, ws, s, err);
    case 2: return launch_wd<8, 1, 2>(gate, up, x, h, rows, nb, ws, s, err);
    case 3: return launch_wd<10, 1, 2>(gate, up, x, h, rows, nb, ws, s, err);
    case 4:
      return lines_fit(nb, gate, up) &&
             launch_wd<6, 2, 2, 1, 4, false, 4, true>(gate, up, x, h, rows, nb, ws, s, err);
    case 5:
      return lines_fit(nb, gate, up) &&
             launch_wd<12, 1, 2, 1, 4, false, 4, true>(gate, up, x, h, rows, nb, ws, s, err);
    default: break;
  }
  // full-line copies at 12 waves: 17408 x 5120 22.9 us against 23.5 (27.7
  // with 6 waves and two stages in flight)
  if (lines_fit(nb, gate, up) &&
      launch_wd<12, 1, 2, 1, 4, false, 4, true>(gate, up, x, h, rows, nb, ws, s, err))
    return true;
  // 12 waves (161 VGPRs, no spills): measured on MI355X against 8, us:
  // 17408 x 5120 23.1 / 24.0, 14336 x 4096 15.5 / 16.6, 11008 x 4096
  // 12.8 / 13.5, 8192 x 2048 6.9 / 7.1-7.4, 4096 x 4096 7.0 / 7.1-7.4
  return launch_wd<12, 1, 2>(gate, up, x, h, rows, nb, ws, s, err) ||
         launch_wd<8, 1, 2>(gate, up, x, h, rows, nb, ws, s, err) ||
         launch_wd<4, 1, 2>(gate, up, x, h, rows, nb, ws, s, err);
}

}  // namespace sihip
