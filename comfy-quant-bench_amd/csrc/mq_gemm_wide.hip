// Large-tile quantized GEMM for gfx950: a TM x TN output tile (256 x 256, 256 x 192 or 128 x 128)
// per workgroup of 8 wavefronts, int8 MFMA (v_mfma_i32_16x16x64_i8: one instruction covers one
// 64-wide K group of a 16 x 16 output tile), one K group per k-step. The 128 tile serves products
// whose 256 tiles would leave most compute units idle (small M); the 256 x 192 tile fills the last
// wave of products such as N = 3072 (16 tile columns instead of 12).
//
// Layout. Waves form a 4 (M) x 2 (N) grid; each owns a TM/4 x TN/2 output tile made of NI x NJ MFMA
// 16x16 tiles (4 x 8, 4 x 6 or 2 x 4). In the 16x16 output layout lane l holds column l % 16 and rows 4 * (l / 16) + r,
// r = 0..3, so every lane needs one weight scale per column tile. A (int8 activation codes) and
// B (weights, unpacked to int8 on their way into LDS) live in a 4-stage LDS ring of 64-byte rows
// whose four 16-byte chunks are XOR-swizzled by (row >> 1) & 3: the fragment reads (lane l reads
// chunk l / 16 of row l % 16) are then free of bank conflicts on gfx950, which a padded pitch of 80
// bytes is not (measured).
//
// Pipeline. The main loop is unrolled over four K groups, so the LDS stage (g % 4) and the sign
// parity (g % 2) of every group are compile-time constants and every LDS access is a base register
// plus an immediate offset. Inside a group the NI NJ MFMA tiles run column by column (t = NI j + i);
// step t issues tile t's MFMA and then the fmas of tile t - 3, so a result is read three MFMAs
// after it was produced while the MFMA and VALU pipes overlap. B fragments sit in a 4-slot
// register ring read three columns ahead; A fragments of group g + 1 are read early in group g.
// A tiles go from HBM to LDS by buffer_load ... lds, three groups ahead; packed B is loaded into
// one of two register sets four groups ahead (inline-asm loads with explicit vmcnt waits), unpacked
// into the stage of group g + 2 mid-group, and one barrier per group closes the ring.
// Zero-points and scales are loaded once per block of four groups (one 2-byte and one 4-byte load
// per weight row), not per group: each such load touches one cache line per row, and per-group
// loads of 1-2 bytes per row were a third of the kernel's L1 -> L2 requests. The scales are stored
// to LDS for the fragment-ordered reads of the fmas, except with expanded weights on 256-row tiles
// (kXS below), whose lanes load their columns' scales from the expansion straight into registers.
//
// Per-group scale epilogue without an int->float conversion. The MFMA accumulator of group g
// is seeded with the bit pattern of 1.5 * 2^23, so the int32 result D = seed + X reads as the
// float 1.5 * 2^23 + X exactly (|X| < 2^22; here |X| <= 64 * 127 * 15). One v_fma_f32 per output
// and group then adds float(D) * s to an fp32 accumulator. To keep the accumulator small (and
// its rounding error at fp32 level) the sign alternates by group: odd groups multiply the
// negated weights (z - q) and add float(D) * (-s). The accumulator then holds
//     sum_g s_g * P_g + 1.5 * 2^23 * sum_g (-1)^g s_g,
// and the second term, accumulated exactly alongside from the same fp32 scales, is removed in the
// final epilogue. The integer partials P_g themselves are exact (GroupPartials writes them).
//
// Weight unpack: packed byte j of a row holds k = 2j in bits 0-3 and k = 2j + 1 in bits 4-7. Four
// bytes at a time: lo/hi nibble masks, (v + (0x80 - z)) ^ 0x80 per byte (no inter-byte carry) for
// q - z, ((0x80 + z) - v) ^ 0x80 for z - q, and two byte permutes back to k order. Signed int4
// is the same with v ^ 8 and z = 8.
//
// int4 activations. With codes in [-7, 7] the partials are ~100x smaller than with int8 codes and
// the fp32 step above would lose accuracy, so int4 operands are scaled by 16 (exact in int8):
// activation layout 1 scales them on their way into LDS; layout 2 (written by the rotate+quantize
// kernel) stores 16 * q negated in odd groups, and signed int4 weights then enter as 16 * v. The
// MFMA result is 2^gshift times the partial (gshift 4 or 8) and the scales are divided by the same
// power of two, so every step stays exact.
#include <algorithm>
#include <type_traits>

#include "mq_device.h"
#include "mq_internal.h"

namespace mq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int TK = 64;
constexpr int LAG = 3;                    // tile t's fmas run LAG MFMAs after it
constexpr int kSeed = 0x4B400000;         // bits of 1.5 * 2^23
constexpr int NSTAGE = 4;

// Tile configuration and LDS map (bytes): 4-stage rings of A tiles, unpacked B tiles and fp32
// scales; the output staging of the epilogue reuses the ring region. The B stages have TM rows like
// the A stages, so every thread keeps the same load and store roles; rows TN .. TM - 1 of a B stage
// (256 x 192 tile) receive only zeros and are never read. 256 tiles: A / B stages of 16 KB, 137 KB
// in all; 128 tile: 8 KB stages, 67.5 KB in all.
constexpr int NT = 512;                                       // threads per workgroup: 8 waves
template <int TM_, int TN_>
struct Cfg {
    static constexpr int TM = TM_, TN = TN_;
    static constexpr int WR = TM / 4, WC = TN / 2;            // wave tile (4 x 2 waves)
    static constexpr int NI = WR / 16, NJ = WC / 16;          // MFMA row / column tiles per wave
    static constexpr int NTL = NI * NJ;                       // MFMA tiles per wave and K group
    static constexpr int NH = TM / 128;                       // 1 KB DMA blocks per wave and K group
    static constexpr int TPR = NT / TM;                       // threads per packed weight row
    static constexpr int BPT = 32 / TPR;                      // packed B bytes per thread and K group
    static constexpr int TILE_BYTES = TM * TK;                // one A or B stage: TM rows x 64 bytes
    static constexpr int A_LDS = 0;
    static constexpr int B_LDS = A_LDS + NSTAGE * TILE_BYTES;
    static constexpr int S_LDS = B_LDS + NSTAGE * TILE_BYTES;
    static constexpr int PIPE_END = S_LDS + NSTAGE * TN * 4;
    static constexpr int OROW = WC + 8;                       // 16-bit pitch of the output staging rows
    static constexpr int OUT_END = (NT / 64) * WR * OROW * 2;
    static constexpr int C_LDS = PIPE_END > OUT_END ? PIPE_END : OUT_END;   // per-column offset correction / fp32 scale
    static constexpr int R_LDS = C_LDS + TN * 4;              // per-row activation scales of the tile
    static constexpr int BI_LDS = R_LDS + TM * 4;             // per-column bias of the tile, as fp32
    static constexpr int SMEM_BYTES = BI_LDS + TN * 4;
};
static_assert(Cfg<256, 256>::SMEM_BYTES <= 160 * 1024 && Cfg<256, 192>::SMEM_BYTES <= 160 * 1024 &&
                  Cfg<128, 128>::SMEM_BYTES <= 160 * 1024, "LDS budget");

// LDS operations a wave issues in a group after its last LDS store (step ts): the B fragment reads
// (steps with i == 0), the next group's A fragment reads and, with group scales, the scale reads
// (steps 3 and 19 for NJ >= 6, step 3 for NJ == 4), in the step schedule of the kernel's group loop.
constexpr int lds_ops_after(int ni, int nj, int ts, bool group_scale) {
    int n = 0;
    for (int t = ts + 1; t < ni * nj; ++t) {
        const int j = t / ni, i = t % ni;
        if (i == 0) ++n;
        if (i == (ni == 4 ? 2 : 1) && j < ni) ++n;
        if (group_scale && (t == 3 || (nj >= 6 && t == 19))) ++n;
    }
    return n;
}

// Tile codes of GemmArgs::tile / choose_tile: the output tile's N extent (256 and 192: 256 rows).
constexpr int tile_rows(int code) { return code == 128 ? 128 : 256; }

// byte offset of 16-byte chunk c of tile row r in the swizzled layout
__device__ __forceinline__ int lds_off(int r, int c) { return r * TK + ((c ^ ((r >> 1) & 3)) << 4); }

// 8 packed 4-bit weights (one dword) -> 8 int8 operands in k order (two dwords). Bytes of c are
// 0x80 - z (u = 0) or 0x80 + z (u = 1): per byte, (lo + c) ^ 0x80 = lo - z and (c - lo) ^ 0x80 =
// z - lo, without inter-byte carries or borrows since lo is in [0, 15].
template <bool NEG>
__device__ __forceinline__ void unpack_nib(uint32_t w, uint32_t c, uint32_t& o0, uint32_t& o1) {
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    if constexpr (NEG) {
        lo = (c - lo) ^ 0x80808080u;
        hi = (c - hi) ^ 0x80808080u;
    } else {
        lo = (lo + c) ^ 0x80808080u;
        hi = (hi + c) ^ 0x80808080u;
    }
    o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

// The per-group constant of unpack_nib for zero-point byte zb (U4Asym) or the fixed zero-point 8
// of signed int4 (whose nibbles are flipped by 8 first, so v ^ 8 = v + 8 is in [0, 15]).
template <WKind WK, bool NEG>
__device__ __forceinline__ uint32_t unpack_const(uint32_t zb) {
    if constexpr (WK == WKind::I4Sym) zb = 8u;
    const uint32_t zz = __builtin_amdgcn_perm(0u, zb, 0u);   // byte 0 of zb in every byte
    return NEG ? (0x80808080u | zz) : (0x80808080u - zz);
}

// U4Asym: q - z (z - q when NEG); I4Sym: v (-v when NEG), or 16 * v when X16 (never negated).
template <WKind WK, bool NEG, bool X16>
__device__ __forceinline__ void unpack_dword(uint32_t w, uint32_t c, uint32_t& o0, uint32_t& o1) {
    if constexpr (WK == WKind::I4Sym && X16) {
        // a nibble moved to the high half of its byte reads as 16 x its signed value
        const uint32_t lo = (w << 4) & 0xf0f0f0f0u, hi = w & 0xf0f0f0f0u;
        o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
    } else {
        if constexpr (WK == WKind::I4Sym) w ^= 0x88888888u;
        unpack_nib<NEG>(w, c, o0, o1);
    }
}

// Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a contiguous range of
// tiles, then order tiles in bands of 4 tile-rows so concurrently resident workgroups on one XCD
// share A rows and B columns in that XCD's L2.
__device__ __forceinline__ void map_tile(int pid, int tiles_m, int tiles_n, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    if (total % 8 == 0) pid = (pid % 8) * (total / 8) + pid / 8;
    constexpr int GM = 4;
    const int in_group = GM * tiles_n;
    const int first_m = (pid / in_group) * GM;
    const int gsize = min(tiles_m - first_m, GM);
    tm = first_m + (pid % in_group) % gsize;
    tn = (pid % in_group) / gsize;
}

// acc = fma(d, (neg ? -1 : 1) * fp16 half `hi` of s, acc) in one v_fma_mix_f32 with the accumulator
// as destination (the compiler's own form leaves the destination free, and the loop's four unrolled
// groups then end with the accumulators in other registers, restored by ~100 moves per iteration).
__device__ __forceinline__ void fma_mix(float& acc, float d, uint32_t s, int hi, int neg) {
    if (hi == 0 && neg == 0) asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(d), "v"(s));
    else if (hi == 0) asm("v_fma_mix_f32 %0, %1, -%2, %0 op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(d), "v"(s));
    else if (neg == 0) asm("v_fma_mix_f32 %0, %1, %2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(d), "v"(s));
    else asm("v_fma_mix_f32 %0, %1, -%2, %0 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "+v"(acc) : "v"(d), "v"(s));
}

// Buffer resource over [base, base + bytes): loads whose vector offset lies outside the range
// return 0 (the scalar offset is added to the address but is not part of that check, so it must
// keep every in-range access inside the buffer). Invalid rows are given the vector offset kOob.
constexpr int kOob = static_cast<int>(0x80000000u);
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                            static_cast<int>(bytes), 0x00020000);
}

// Buffer loads written as inline asm, so that the kernel alone decides when to wait for them
// (s_waitcnt vmcnt with counts that follow the pipeline's fixed issue order; the compiler's own
// count is conservative at the loop header and would wait for loads issued a group later).
// The descriptor is the same as make_buffer_rsrc builds: base, stride 0, byte range, format word.
// Each load starts with s_nop 4: the compiler may have just restored the descriptor or the scalar
// offset from a VGPR lane (v_readlane), and a VMEM instruction reading an SGPR written by VALU
// needs 5 wait states, which the compiler does not insert in front of inline asm.
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u4v sdesc(const void* base, int64_t bytes) {
    const uint64_t p = reinterpret_cast<uint64_t>(base);
    u4v d;
    d.x = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
    d.y = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32) & 0xffffu);
    d.z = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bytes));
    d.w = 0x00020000u;
    return d;
}
__device__ __forceinline__ u4v asm_ld128(u4v d, int voff, int soff) {
    u4v v;
    asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(d), "s"(soff) : "memory");
    return v;
}
typedef uint32_t u2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u2v asm_ld64(u4v d, int voff, int soff) {
    u2v v;
    asm volatile("s_nop 4\n\tbuffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(d), "s"(soff) : "memory");
    return v;
}
typedef uint32_t u3v __attribute__((ext_vector_type(3)));
__device__ __forceinline__ u3v asm_ld96(u4v d, int voff, int soff) {
    u3v v;
    asm volatile("s_nop 4\n\tbuffer_load_dwordx3 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(d), "s"(soff) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t asm_ld32(u4v d, int voff, int soff) {
    uint32_t v;
    asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(d), "s"(soff) : "memory");
    return v;
}
__device__ __forceinline__ uint32_t asm_ld16(u4v d, int voff, int soff) {
    uint32_t v;
    asm volatile("s_nop 4\n\tbuffer_load_ushort %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(d), "s"(soff) : "memory");
    return v;
}

// 16 bytes per lane from buffer r at voff + soff straight into LDS: lane l writes bytes
// [lds_off + 16 l, lds_off + 16 l + 16) (lds_off is wave-uniform; it becomes M0).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* smem, int lds_off, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(smem + lds_off), 16, voff,
                                             soff, 0, 0);
}

// LDS stores written as inline asm. The compiler orders every LDS access after a pending LDS DMA
// (buffer_load ... lds) by waiting for the DMA to complete; these stores never alias a DMA in
// flight (different ring region or stage), and their completion is awaited explicitly. imm is
// stage * STRIDE (stage 0..3, known once inlined), taken as the instruction's immediate offset.
template <int STRIDE>
__device__ __forceinline__ void ds_write16(int base, int imm, uint4 v) {
    typedef uint32_t u4v __attribute__((ext_vector_type(4)));
    const u4v x = {v.x, v.y, v.z, v.w};
    if (imm == 0) asm volatile("ds_write_b128 %0, %1" ::"v"(base), "v"(x) : "memory");
    else if (imm == STRIDE) asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(base), "v"(x), "n"(STRIDE) : "memory");
    else if (imm == 2 * STRIDE) asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(base), "v"(x), "n"(2 * STRIDE) : "memory");
    else asm volatile("ds_write_b128 %0, %1 offset:%2" ::"v"(base), "v"(x), "n"(3 * STRIDE) : "memory");
}
template <int STRIDE>
__device__ __forceinline__ void ds_write4(int base, int imm, float v) {
    if (imm == 0) asm volatile("ds_write_b32 %0, %1" ::"v"(base), "v"(v) : "memory");
    else if (imm == STRIDE) asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(base), "v"(v), "n"(STRIDE) : "memory");
    else if (imm == 2 * STRIDE) asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(base), "v"(v), "n"(2 * STRIDE) : "memory");
    else asm volatile("ds_write_b32 %0, %1 offset:%2" ::"v"(base), "v"(v), "n"(3 * STRIDE) : "memory");
}

template <typename T>
__device__ __forceinline__ T& lds(uint8_t* smem, int off) {
    return *reinterpret_cast<T*>(smem + off);
}

// One workgroup: a T x T output tile. AM is the activation layout of the group epilogues
// (0 int8 codes; 2 int4 codes stored as 16 * q and negated in odd groups, signed int4 weights then
// entering as 16 * v); row epilogues use 0. XP (4-bit kinds, group scales): the weights come
// expanded to int8 in 16-row tiles (mq_expand_weight_w4: the bytes the unpack would store, zero-point
// and sign included), so B takes A's DMA path and no zero-points are loaded; the arithmetic, and
// the scaling by WK and AM, is the packed kernel's.
template <int TM_, int TN_, WKind WK, Epi EPI, int AM, bool SPLIT, bool XP>
__global__ void __launch_bounds__(NT) gemm_wide_kernel(GemmArgs a, int tiles_m, int tiles_n) {
    using C = Cfg<TM_, TN_>;
    constexpr int TM = C::TM, TN = C::TN, NI = C::NI, NJ = C::NJ, NTL = C::NTL, TILE_BYTES = C::TILE_BYTES;
    constexpr int WR = C::WR, WC = C::WC, NH = C::NH, TPR = C::TPR;
    constexpr int A_LDS = C::A_LDS, B_LDS = C::B_LDS, S_LDS = C::S_LDS, OROW = C::OROW;
    constexpr int C_LDS = C::C_LDS, R_LDS = C::R_LDS, BI_LDS = C::BI_LDS;
    static_assert(!SPLIT || EPI == Epi::GroupScale || EPI == Epi::RowScale, "split-K outputs partial results");
    static_assert(AM == 0 || AM == 2, "activation layout 1 is served by the 128-tile kernel");
    constexpr bool kGroup = EPI == Epi::GroupScale || EPI == Epi::GroupPartials;
    static_assert(!XP || (WK != WKind::I8 && EPI == Epi::GroupScale), "expanded 4-bit weights, group scales");
    constexpr bool kPacked = WK != WKind::I8 && !XP;
    constexpr bool kHasZ = WK == WKind::U4Asym && !XP;   // zero-points loaded (packed uint4 weights)
    constexpr int kShift = kGroup && AM == 2 ? (WK == WKind::I4Sym ? 8 : 4) : 0;
    constexpr float kSfac = 1.0f / static_cast<float>(1 << kShift);
    // kXS (expanded weights on 256-row tiles): the expanded weights carry their group scales as fp16
    // column pairs after the int8 tiles (mq_expand_weight_w4: dword [g][c][u] = the scales of group
    // g of columns 32 u + c and 32 u + 16 + c, zero past N and past G, scale_pair_ld(N) dwords per
    // [g][c] row). Each lane loads its NJ columns' scales of a group with one load straight into
    // registers (no LDS stores or reads, no LDS wait before the group's barrier), one group ahead,
    // and the fp32 step multiplies by the fp16 scale itself (v_fma_mix). The step then runs unscaled
    // by kSfac, a power of two moved to the row scales of the epilogue: every product and sum is
    // 2^kShift times the scaled one, the same bits after it. The 128 x 128 tile keeps its scales in
    // LDS (its eight-MFMA groups leave a load one group ahead too little time: 25 % slower; loads
    // three groups ahead in four register slots were still 5 % slower than the LDS scales).
    constexpr bool kXS = XP && TM_ == 256;
    constexpr float kSfacA = kXS ? kSfac : 1.0f;   // applied to the activation scales
    __shared__ __attribute__((aligned(16))) uint8_t smem[C::SMEM_BYTES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    const int tiles = tiles_m * tiles_n;
    const int slice = SPLIT ? static_cast<int>(blockIdx.x) / tiles : 0;
    map_tile(SPLIT ? static_cast<int>(blockIdx.x) % tiles : static_cast<int>(blockIdx.x), tiles_m, tiles_n, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * TM, n0 = static_cast<int64_t>(tn) * TN;
    const int64_t M = a.M, N = a.N;
    const int G = static_cast<int>(a.K / TK);
    const int G4 = (G + 3) / 4 * 4;   // groups run, live and dead
    // this workgroup's K groups [g0, g1) (all of them without split-K); g0 % 4 == 0
    const int g0 = SPLIT ? slice * a.kgroups : 0;
    const int g1 = SPLIT ? min(g0 + a.kgroups, G4) : G4;
    const int gend = min(g1, G);      // groups whose products this workgroup accumulates
    const int rows_m = M - m0 < TM ? static_cast<int>(M - m0) : TM;   // valid rows of this tile
    const int rows_n = N - n0 < TN ? static_cast<int>(N - n0) : TN;
    const int kbytes_w = kPacked ? static_cast<int>(a.K / 2) : static_cast<int>(a.K);
    // The output epilogue's per-row and per-column inputs (activation scales, bias, fp32 weight
    // scales), loaded now and put into LDS once the prologue's loads have landed, so the epilogue
    // reads them from LDS: thread t < TM takes row m0 + t, thread TM + c column n0 + c. Rows and
    // columns past the matrix get 0.
    constexpr bool kFinal = !SPLIT && (EPI == Epi::GroupScale || EPI == Epi::RowScale);
    float ep_a = 0.0f, ep_b = 0.0f;
    if constexpr (kFinal) {
        if (tid < TM) {
            if (tid < rows_m) ep_a = a.sa[m0 + tid] * kSfacA;   // exact
        } else if (tid - TM < rows_n) {
            const int64_t col = n0 + (tid - TM);
            if (a.bias) ep_a = load_as_f32(a.bias, a.bias_dtype, col);
            if constexpr (EPI == Epi::RowScale) ep_b = a.ws32[col];
        }
    }
    // activation codes in 16-row tiles (the linears' own codes): whole-line DMA rows, as for B
    const bool at = a.atile;
    const auto ra_rs = at ? rsrc(a.qa + (m0 >> 4) * G * 1024, static_cast<int64_t>((rows_m + 15) >> 4) * G * 1024)
                          : rsrc(a.qa + m0 * a.lda, (rows_m - 1) * a.lda + a.K);
    // int8 weights in 16-row tiles: the K group of 16 rows is one 1 KB block, so every DMA
    // instruction reads whole 128-byte lines (rows of ldw bytes give it two halves of 16 lines)
    const bool wt = !kPacked && a.wtile;
    const auto rb_rs = wt ? rsrc(a.qw + (n0 >> 4) * G * 1024, static_cast<int64_t>((rows_n + 15) >> 4) * G * 1024)
                          : rsrc(a.qw + n0 * a.ldw, (rows_n - 1) * a.ldw + kbytes_w);

    // ---- DMA roles (A, and int8 B): wave w copies tile rows [16 NH w, 16 NH (w + 1)) of a K group
    // as NH 1 KB blocks. Lane l of block h writes LDS bytes [16 l, 16 l + 16) of tile row
    // 16 NH w + 16 h + l / 4; that is physical chunk l % 4 of the swizzled row, so it fetches
    // logical chunk (l % 4) ^ swizzle(row).
    int dma_a[NH], dma_b[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
        const int r = 16 * NH * wave + 16 * h + (lane >> 2);
        const int c = (lane & 3) ^ ((r >> 1) & 3);
        dma_a[h] = r >= rows_m ? kOob
                   : at ? (r >> 4) * G * 1024 + (r & 15) * 64 + c * 16
                        : static_cast<int>(r * a.lda) + c * 16;
        dma_b[h] = r >= rows_n ? kOob
                   : wt ? (r >> 4) * G * 1024 + (r & 15) * 64 + c * 16
                        : static_cast<int>(r * a.ldw) + c * 16;
    }
    const int dma_lds = (16 * NH * wave) * TK;   // + 16 * TK for block h

    // ---- packed B roles: TPR threads per weight row (2 for T = 256, 4 for T = 128), 32 / TPR packed
    // bytes (64 / TPR weights, 16-byte LDS chunks 2 bpart and 2 bpart + 1, or chunk bpart) each; the
    // threads with bpart < 2 also carry the row's scales (bhalf = bpart)
    const int brow = tid / TPR, bpart = tid % TPR, bhalf = bpart & 1;
    const bool b_ok = brow < rows_n;
    const int b_off = b_ok ? static_cast<int>(brow * a.ldw) + bpart * C::BPT : kOob;
    // zero-points and scales (null for the kinds that have none: the range is then empty)
    const bool has_z = kHasZ, has_s = EPI == Epi::GroupScale;
    const u4v db = sdesc(a.qw + n0 * a.ldw, (rows_n - 1) * a.ldw + kbytes_w);
    const u4v dz = sdesc(has_z ? a.wz + n0 * a.ldwz : a.qw, has_z ? (rows_n - 1) * a.ldwz + (G + 1) / 2 : 0);
    const u4v ds = sdesc(has_s ? static_cast<const void*>(a.ws16 + n0 * a.ldws) : a.qw,
                         has_s ? ((rows_n - 1) * a.ldws + G) * 2 : 0);
    const int z_off = has_z && b_ok ? static_cast<int>(brow * a.ldwz) : kOob;
    const int s_off = has_s && b_ok && bpart < 2 ? static_cast<int>(brow * a.ldws * 2) + 4 * bhalf : kOob;
    // kXS: the scale pairs after the expanded weight's tiles, G4 groups (every access below lies
    // inside them)
    const int sp_ld = static_cast<int>(scale_pair_ld(N));                 // dwords per [g][c] row
    const int sp_stride = 16 * sp_ld * 4;                                  // bytes per group
    const auto rsp = rsrc(a.qw + (N + 15) / 16 * 16 * a.K, kXS ? static_cast<int64_t>(G4) * sp_stride : 0);
    const auto rsp_none = rsrc(a.qw, 0);
    const int b_st00 = B_LDS + lds_off(brow, TPR == 2 ? 2 * bpart : bpart);
    const int b_st10 = B_LDS + lds_off(brow, TPR == 2 ? 2 * bpart + 1 : bpart);
    // scales stored transposed, [wn][column % 16][column tile], so a lane's NJ scales are adjacent
    const int s_st0 = S_LDS + 4 * ((((brow / WC) * 16) + (brow & 15)) * NJ + ((brow % WC) >> 4));

    // fragment reads: lane l reads chunk l / 16 of row l % 16 of a 16-row block (swizzle depends
    // only on the row within the block, so one per-lane offset serves every block)
    const int fr = lane & 15, fk = ((lane >> 4) ^ ((fr >> 1) & 3)) << 4;
    // kXS: this lane's scales, columns n0 + wn WC + 16 j + fr, j = 0 .. NJ - 1, in NJ / 2 adjacent
    // dwords (n0 + wn WC is a multiple of 32)
    const int sc_off = static_cast<int>((fr * sp_ld + ((n0 + wn * WC) >> 5)) * 4);
    const int a_rd0 = A_LDS + (wm * WR + fr) * TK + fk;   // + i * 16 * TK
    const int b_rd0 = B_LDS + (wn * WC + fr) * TK + fk;   // + j * 16 * TK
    const int s_rd0 = S_LDS + 4 * ((wn * 16 + fr) * NJ);        // + 4 * j
    // opaque LDS base registers: every access below is base + a compile-time offset below 64 KB,
    // which the ds instructions take as an immediate
    int a_rd = a_rd0, b_rd = b_rd0, s_rd = s_rd0, b_st0 = b_st00, b_st1 = b_st10, s_st = s_st0;
    asm volatile("" : "+v"(a_rd), "+v"(b_rd), "+v"(s_rd), "+v"(b_st0), "+v"(b_st1), "+v"(s_st));

    // Groups past the last one ("dead" groups, which pad the loop to a multiple of the unroll) load
    // through resources of zero bytes, so every such access is out of range and returns 0: their
    // codes, zero-points and scales are all zero and add nothing to any accumulator. (A scalar
    // offset past the range would not do: the range check does not include it.)
    const auto ra_none = rsrc(a.qa, 0);
    const auto rb_none = rsrc(a.qw, 0);
    const u4v d_none = sdesc(a.qw, 0);
    auto soff = [&](int g, int per_group) { return g < G ? g * per_group : 0; };
    // DMA of group g's A (and int8 B) tile into stage st
    auto dma_group = [&](int g, int st) {
        const bool live = g < G;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            dma16(live ? ra_rs : ra_none, smem, A_LDS + st * TILE_BYTES + dma_lds + h * 16 * TK, dma_a[h],
                  soff(g, at ? 1024 : TK));
            if constexpr (!kPacked)
                dma16(live ? rb_rs : rb_none, smem, B_LDS + st * TILE_BYTES + dma_lds + h * 16 * TK, dma_b[h],
                      soff(g, wt ? 1024 : TK));
        }
    };
    // Two register sets carry packed B groups from their global load to their LDS store.
    using BV = std::conditional_t<TPR == 2, u4v, u2v>;
    BV rb[2] = {BV{}, BV{}};
    auto gload_b = [&](int g, int set) {
        if constexpr (kPacked) {
            if constexpr (TPR == 2) rb[set] = asm_ld128(g < G ? db : d_none, b_off, soff(g, TK / 2));
            else rb[set] = asm_ld64(g < G ? db : d_none, b_off, soff(g, TK / 2));
        }
    };
    // Zero-points and scales of a block of four K groups b4 .. b4 + 3 (b4 % 4 == 0), one load each
    // per block instead of one per group: zq holds the four zero-point nibbles (group b4 + u in
    // bits 4u .. 4u + 3), sq the fp16 scales of groups b4 + 2 bhalf and b4 + 2 bhalf + 1. Groups
    // past the last one read zero or another row's values; their scales are zeroed at the store
    // and their activations are zero.
    // The tile's last weight row has nothing after its ceil(G/2) zero-point bytes and G scales
    // inside the resource range (the range check covers the vector offset only): in the block that
    // runs past G (G % 4 != 0) that row's loads move back to end at the row's end (or, for a scale
    // pair wholly past G, fail the range check), and the bytes they want are shifted down once the
    // loads have arrived (settle_zs, by zsh / ssh bits). The host keeps G >= 3 on this kernel, so
    // moving back stays inside the row.
    // Only the last live block (b4 = 4 * ((G - 1) / 4)) can run past G; its offsets and shifts are
    // worked out once here.
    const bool last_row = brow == rows_n - 1;
    const int last_b4 = (G - 1) / 4 * 4;
    int z_last = z_off, s_last = s_off;
    uint32_t zsh_last = 0u, ssh_last = 0u;
    if (last_row && z_off != kOob && last_b4 / 2 + 2 > (G + 1) / 2) {
        z_last = z_off - 1;
        zsh_last = 8u;
    }
    if (last_row && s_off != kOob) {
        const int ga = last_b4 + 2 * bhalf;   // first group of this thread's scale pair
        if (ga >= G) s_last = kOob;
        else if (ga + 1 == G) {
            s_last = s_off - 2;
            ssh_last = 16u;
        }
    }
    uint32_t zq = 0u, sq = 0u, zsh = 0u, ssh = 0u;
    // once a block's zero-points and scales have arrived (before their first use): the moved-back
    // loads of the last block bring the wanted bytes down
    auto settle_zs = [&]() {
        if constexpr (kHasZ) zq >>= zsh;
        if constexpr (EPI == Epi::GroupScale) sq >>= ssh;
    };
    auto gload_zs = [&](int b4) {
        const bool lb = b4 == last_b4;   // wave-uniform
        if constexpr (kHasZ) {
            zsh = lb ? zsh_last : 0u;
            zq = asm_ld16(b4 < G ? dz : d_none, lb ? z_last : z_off, b4 < G ? b4 >> 1 : 0);
        }
        if constexpr (EPI == Epi::GroupScale) {
            ssh = lb ? ssh_last : 0u;
            sq = asm_ld32(b4 < G ? ds : d_none, lb ? s_last : s_off, soff(b4, 2));
        }
    };
    // kXS: group g's scales of this lane's NJ columns into register slot `slot` (= g % 2); groups
    // past the scale pairs (the loop's last loads) read zeros through an empty range
    uint32_t sc[2][NJ / 2];
#pragma unroll
    for (int h = 0; h < NJ / 2; ++h) sc[0][h] = sc[1][h] = 0u;
    auto gload_sc = [&](int g, int slot) {
        if constexpr (kXS) {
            const auto r = g < G4 ? rsp : rsp_none;
            const int so = g < G4 ? g * sp_stride : 0;
            if constexpr (NJ == 8) {
                const v4i v = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, sc_off, so, 0));
                sc[slot][0] = v.x; sc[slot][1] = v.y; sc[slot][2] = v.z; sc[slot][3] = v.w;
            } else if constexpr (NJ == 6) {
                const u3v v = __builtin_amdgcn_raw_buffer_load_b96(r, sc_off, so, 0);
                sc[slot][0] = v.x; sc[slot][1] = v.y; sc[slot][2] = v.z;
            } else {
                static_assert(NJ == 4, "tiles of 4, 6 or 8 column blocks per wave");
                const u2v v = __builtin_amdgcn_raw_buffer_load_b64(r, sc_off, so, 0);
                sc[slot][0] = v.x; sc[slot][1] = v.y;
            }
        }
    };
    // kXS: a wait for at most N outstanding VMEM operations before the barrier (the compiler also
    // waits for each scale load itself before its first use; these loads are visible to it)
    auto wait_sc = [&](auto Nc, auto) {
        if constexpr (kXS) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(decltype(Nc)::value) : "memory");
    };
    // Wait until at most N VMEM operations are outstanding; register set SET counts as written by
    // the wait, so no use of it moves above it.
#define MQ_WAIT_B(N, SET) \
    asm volatile("s_waitcnt vmcnt(%3)" : "+v"(rb[SET]), "+v"(zq), "+v"(sq) : "n"(N) : "memory")
    // sum_g (-1)^g s[n, g] over the groups whose scale this thread stores (half of them: threads
    // bpart 0 and 1 of a weight row, adjacent lanes, add their sums in the epilogue)
    float cs = 0.0f;
    // LDS stores of register set `set` (a group of parity PAR) into stage ST, in two halves of the
    // unpacked row (spread over two steps) and the scale.
    // PARc: parity of the group stored, Uc: its position in its block of four (u = g % 4)
    auto store_b = [&](int st, int set, auto PARc, auto Uc, int h) {
        if constexpr (kPacked) {
            constexpr bool neg = kGroup && decltype(PARc)::value == 1;
            constexpr bool x16 = AM == 2 && kGroup;
            constexpr bool nw = neg && AM != 2;
            constexpr int pos = decltype(Uc)::value;
            const uint32_t c = unpack_const<WK, nw>((zq >> (4 * pos)) & 0xfu);
            uint4 u;
            uint32_t w0 = rb[set].x, w1 = rb[set].y;
            if constexpr (TPR == 2) {
                if (h) {
                    w0 = rb[set].z;
                    w1 = rb[set].w;
                }
            }
            unpack_dword<WK, nw, x16>(w0, c, u.x, u.y);
            unpack_dword<WK, nw, x16>(w1, c, u.z, u.w);
            ds_write16<TILE_BYTES>(h ? b_st1 : b_st0, st * TILE_BYTES, u);
        }
    };
    // scale of group g (position u in its block) by the thread of its row that loaded it
    auto store_s = [&](int st, int g, auto PARc, auto Uc) {
        if constexpr (EPI == Epi::GroupScale) {
            constexpr bool neg = decltype(PARc)::value == 1;
            constexpr int u = decltype(Uc)::value;
            if (bpart == (u >> 1) && (TN == TM || brow < TN)) {
                float sv = f16_bits_to_f32(static_cast<uint16_t>(sq >> (16 * (u & 1)))) * (kXS ? 1.0f : kSfac);   // exact
                sv = g >= g0 && g < gend ? (neg ? -sv : sv) : 0.0f;
                if constexpr (!kXS) ds_write4<TN * 4>(s_st, st * TN * 4, sv);
                cs += sv;
            }
        }
    };

    float acc[NI][NJ][4];
    v4i acci[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[i][j][r] = 0.0f;
                acci[i][j][r] = 0;
            }
        }

    // Fragment registers: A fragments of the current and the next K group (set = g % 2), a 4-slot
    // ring of B fragments read three columns ahead (slot = running column count % 4), the column scales in two
    // register quads (NJ = 8: columns 0-3 and 4-7 of a group; NJ = 4: the four columns of the groups
    // of parity 0 and 1), and a 4-slot ring of MFMA results (slot = tile % 4). The ring slots a
    // tile or column uses are the same in every group, so the pipeline state at a group boundary
    // does not depend on which unrolled copy ran last. Zeroed results and scales make the first
    // group's look-back fmas add nothing.
    v4i fa[2][NI], fb[4], d[4];
    f4 fs[2] = {f4{0.0f, 0.0f, 0.0f, 0.0f}, f4{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int q = 0; q < 4; ++q) d[q] = v4i{0, 0, 0, 0};
    const v4i seed = {kSeed, kSeed, kSeed, kSeed};
    auto read_a = [&](int st, int set, int i) { fa[set][i] = lds<v4i>(smem, a_rd + st * TILE_BYTES + i * 16 * TK); };
    // B column col of a stage into ring slot `slot`: the slot of column j of group g is
    // (g NJ + j) % 4, a running column count, so the ring wraps across groups for every NJ
    auto read_b = [&](int st, int col, int slot) { fb[slot] = lds<v4i>(smem, b_rd + st * TILE_BYTES + col * 16 * TK); };
    // the 4 scales of columns 4 h .. 4 h + 3 (adjacent in the transposed scale layout) into quad q
    auto read_s = [&](int st, int h, int q) {
        if constexpr (EPI == Epi::GroupScale && !kXS) fs[q] = lds<f4>(smem, s_rd + st * TN * 4 + 16 * h);
    };
    // Partials of tile tp (held in d[tp & 3]) of group gp.
    auto write_partials = [&](int tp, int gp, bool odd) {
        const int ip = tp % NI, jp = tp / NI;
        const int64_t col = n0 + wn * WC + jp * 16 + fr;
        int32_t* part = a.part + static_cast<int64_t>(gp) * M * N;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = m0 + wm * WR + ip * 16 + 4 * (lane >> 4) + r;
            const int32_t pv = (d[tp & 3][r] - kSeed) >> kShift;   // exact: a multiple of 2^kShift
            if (row < M && col < N) part[row * N + col] = odd ? -pv : pv;
        }
    };
    // fmas of tile tp of a group of parity par: acc += float(seed + X) * (+-s); kXS: s is the tile
    // column's fp16 scale in slot par, taken as fp16 by the fma itself (v_fma_mix_f32)
    auto fma_tile = [&](int tp, int par) {
        const int ip = tp % NI, jp = tp / NI;
        if constexpr (kXS) {
            const uint32_t sp = sc[par][jp >> 1];
#pragma unroll
            for (int r = 0; r < 4; ++r) fma_mix(acc[ip][jp][r], __int_as_float(d[tp & 3][r]), sp, jp & 1, par);
            return;
        }
        const float sv = NJ >= 6 ? fs[jp >> 2][jp & 3] : fs[par][jp & 3];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            acc[ip][jp][r] = __builtin_fmaf(__int_as_float(d[tp & 3][r]), sv, acc[ip][jp][r]);
        asm volatile("" : "+v"(acc[ip][jp][0]), "+v"(acc[ip][jp][1]), "+v"(acc[ip][jp][2]), "+v"(acc[ip][jp][3]));
    };

    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // Prologue. Steady state at the start of group g: A(g), A(g + 1) (and int8 B) complete in
    // stages g % 4, (g + 1) % 4 and A(g + 2) in flight; B(g), B(g + 1) unpacked in their stages;
    // register set g % 2 holds (or is loading) B(g + 2), set (g + 1) % 2 B(g + 3).
    // The VMEM issue order leaves B(2), A(2), B(3) in flight, as in the steady state; A(0), A(1) are
    // complete once the compiler has waited for B(1)'s registers.
    gload_sc(g0, 0);   // kXS: the first group's scales (each group loads the next one's)
    dma_group(g0, 0);
    dma_group(g0 + 1, 1);
    gload_zs(g0);
    gload_b(g0, 0);
    gload_b(g0 + 1, 1);
    MQ_WAIT_B(0, 0);
    MQ_WAIT_B(0, 1);
    wait_sc(I0{}, std::integral_constant<int, 0>{});
    settle_zs();
    store_b(0, 0, I0{}, I0{}, 0);
    store_b(0, 0, I0{}, I0{}, 1);
    store_s(0, g0, I0{}, I0{});
    store_b(1, 1, I1{}, I1{}, 0);
    store_b(1, 1, I1{}, I1{}, 1);
    store_s(1, g0 + 1, I1{}, I1{});
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // A(0), A(1) of every kind (int8 B has no B loads)
    if constexpr (kFinal) {
        if (tid < TM) {
            lds<float>(smem, R_LDS + 4 * tid) = ep_a;
        } else if (tid - TM < TN) {
            lds<float>(smem, BI_LDS + 4 * (tid - TM)) = ep_a;
            if constexpr (EPI == Epi::RowScale) lds<float>(smem, C_LDS + 4 * (tid - TM)) = ep_b;
        }
    }
    gload_b(g0 + 2, 0);
    dma_group(g0 + 2, 2);
    gload_b(g0 + 3, 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < NI; ++i) read_a(0, 0, i);
    read_b(0, 0, 0);
    read_b(0, 1, 1);
    read_b(0, 2, 2);
    read_s(0, 0, 0);
    if constexpr (NJ >= 6) read_s(0, 1, 1);

    // VMEM instructions per group and thread, in issue order: the DMA of A(g + 3) (and int8 B) at
    // step kTD, the packed B load of group g + 4 at step kTL and, in groups with g % 4 == 1, the
    // zero-points and scales of the block g + 3 .. g + 6 right after it. Waits count the VMEM
    // operations issued after the one awaited. With int8 weights the group's DMA is all its VMEM
    // work; issued eight MFMAs into the group rather than at its first, it takes 1.5-2 % off the
    // 256 x 256 row-scale product (measured, same bits).
    // kXS: group g + 1's scales load at step LAG of group g (once group g - 1's last fmas, steps
    // 0 .. LAG - 1, have read that slot), ahead of the group's DMA; the wait before the barrier that
    // ends group g takes them (kTD > LAG).
    constexpr int kDmaOps = NH * (kPacked ? 1 : 2);
    constexpr int kTD = kPacked ? 0 : kXS && 8 % NTL <= LAG ? LAG + 1 : 8 % NTL;
    static_assert(!kXS || kTD > LAG, "the scales load before the group's DMA");
    // steps of the B unpack (kTB: wait for the registers, store; kTB + 1: second half for T = 256),
    // of the scale store (kTS) and of the next packed B load (kTL); kTB > 0 follows the DMA of step 0
    // (packed weights)
    constexpr int kTB = NTL >= 24 ? 8 : 4, kTS = NTL >= 24 ? 10 : 5, kTL = NTL >= 24 ? 12 : 6;
    constexpr int kB = kPacked ? 1 : 0;
    constexpr int kZS = kHasZ + (EPI == Epi::GroupScale);
    // Before the barrier that ends group g, A(g + 2) (issued at step kTD of group g - 1) must be
    // complete; issued after it: B(g + 3), [zs if (g - 1) % 4 == 1], A(g + 3), B(g + 4),
    // [zs if g % 4 == 1]. (The partials variant also stores to global memory; it waits for all.)
    // kXS: group g + 1's scales (issued at step LAG of group g, before its DMA and zs) must be complete
    // too, which leaves only the group's DMA and zs outstanding.
    constexpr int kVmAfter[4] = {
        EPI == Epi::GroupPartials ? 0 : kDmaOps + 2 * kB,
        EPI == Epi::GroupPartials ? 0 : kDmaOps + 2 * kB + kZS,
        EPI == Epi::GroupPartials ? 0 : kXS ? kDmaOps : kDmaOps + 2 * kB + kZS,
        EPI == Epi::GroupPartials ? 0 : kDmaOps + 2 * kB};
    // At step kTB of group g, register set g % 2 (B(g + 2), loaded at step kTL of group g - 2) must
    // have arrived, and in groups with g % 4 == 2 the block of zero-points and scales loaded at the
    // end of group g - 1. Issued after B(g + 2): [zs if g % 4 == 3], A(g + 2), B(g + 3),
    // [zs if g % 4 == 2], A(g + 3).
    // kXS has no B registers: only the block's scales (g % 4 == 2) are awaited, with the group's scale
    // load and DMA issued after them.
    constexpr int kWaitB[4] = {
        EPI == Epi::GroupPartials ? 0 : kXS ? 63 : 2 * kDmaOps + kB,
        EPI == Epi::GroupPartials ? 0 : kXS ? 63 : 2 * kDmaOps + kB,
        EPI == Epi::GroupPartials ? 0 : kXS ? 1 + kDmaOps : (kZS > 0 ? kDmaOps : 2 * kDmaOps + kB),
        EPI == Epi::GroupPartials ? 0 : kXS ? 63 : 2 * kDmaOps + kB + kZS};

    // K group g with A stage, B stage and register set fixed by U = g % 4 (compile-time). Step t = NI j + i.
    auto group = [&](int g, auto Uc) {
        constexpr int U = decltype(Uc)::value;
        constexpr int ST = U, ST1 = (U + 1) % 4, ST2 = (U + 2) % 4, ST3 = (U + 3) % 4, SET = U % 2;
        using PARc = std::integral_constant<int, U % 2>;
        using U2c = std::integral_constant<int, (U + 2) % 4>;   // position of group g + 2 in its block
        constexpr int PAR = PARc::value;
#pragma unroll
        for (int t = 0; t < NTL; ++t) {
            const int j = t / NI, i = t % NI;
            if constexpr (kGroup) {
                d[t & 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[SET][i], fb[(PAR * NJ + j) & 3], seed, 0, 0, 0);
            } else {
                asm volatile("" : "+a"(acci[i][j]));
                acci[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[SET][i], fb[(PAR * NJ + j) & 3], acci[i][j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            // tile t - LAG (for t < LAG: the last tiles of the previous group)
            const int tp = (t + NTL - LAG) % NTL;
            if constexpr (EPI == Epi::GroupScale) fma_tile(tp, t < LAG ? PAR ^ 1 : PAR);
            if constexpr (EPI == Epi::GroupPartials) {
                const int gp = t < LAG ? g - 1 : g;
                if (gp >= 0 && gp < G) write_partials(tp, gp, t < LAG ? PAR == 0 : PAR == 1);
            }
            if constexpr (kXS)
                if (t == LAG) gload_sc(g + 1, PAR ^ 1);
            if (t == kTD) dma_group(g + 3, ST3);
            // B fragments three columns ahead (the next group's first columns from stage ST1,
            // complete since the barrier that ended group g - 1)
            if (i == 0) {
                if (j + 3 < NJ) read_b(ST, j + 3, (PAR * NJ + j + 3) & 3);
                else read_b(ST1, j + 3 - NJ, (PAR * NJ + j + 3) & 3);
            }
            // Scales. NJ = 8: columns 4-7 once the previous group's column 7 is done (its last fma
            // is at step 2), columns 0-3 of the next group once column 3 is done (last fma at step
            // 18). NJ = 4: the next group's columns into the quad of its parity once the previous
            // group's last fma (step 2) has read that quad.
            if constexpr (NJ >= 6) {
                if (t == 3) read_s(ST, 1, 1);
                if (t == 19) read_s(ST1, 0, 0);
            } else {
                if (t == 3) read_s(ST1, 0, PAR ^ 1);
            }
            // the next group's A fragments into the other set, early in this group
            if (i == (NI == 4 ? 2 : 1) && j < NI) read_a(ST1, SET ^ 1, j);
            // unpack register set SET (group g + 2, parity PAR) into stage ST2, then reload it with g + 4
            if (t == kTB) {
                MQ_WAIT_B(kWaitB[U], SET);
                // group g + 2 opens the block of zero-points and scales loaded in group g - 1
                if constexpr (U == 2) settle_zs();
                store_b(ST2, SET, PARc{}, U2c{}, 0);
            }
            if constexpr (TPR == 2)
                if (t == kTB + 1) store_b(ST2, SET, PARc{}, U2c{}, 1);
            if (t == kTS) store_s(ST2, g + 2, PARc{}, U2c{});
            if (t == kTL) {
                gload_b(g + 4, SET);
                if constexpr (U == 1) gload_zs(g + 3);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // A(g + 2) and this group's B stores become visible to every wave. LDS operations of a wave
        // complete in issue order. 256 x 256: the MFMAs of steps 24-27 waited for a fragment read
        // issued after the stores of steps 8-10, so those stores are complete here without a wait.
        // The other tiles: no MFMA of the group reads a fragment issued after the stores, so the
        // wave waits until at most the LDS operations issued after its last store are outstanding
        // (the next group's fragment and scale reads, which stay in flight across the barrier).
        // Group g's own stages were last read by MFMAs that have issued.
        // (kXS: group g + 1's scales, slot PAR ^ 1, arrive with the same wait. kXS stores nothing to LDS
        // in the loop, so no LDS wait is needed.)
        if constexpr (kXS) wait_sc(std::integral_constant<int, kVmAfter[U]>{}, std::integral_constant<int, PAR ^ 1>{});
        else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kVmAfter[U]) : "memory");
        if constexpr (NJ != 8 && !kXS) {
            constexpr int kLdsAfter = lds_ops_after(NI, NJ, kTS, EPI == Epi::GroupScale);
            static_assert(kLdsAfter < 16, "lgkmcnt holds 0-15");
            asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(kLdsAfter) : "memory");
        }
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    for (int g = g0; g < g1; g += 4) {
        group(g, std::integral_constant<int, 0>{});
        group(g + 1, std::integral_constant<int, 1>{});
        group(g + 2, std::integral_constant<int, 2>{});
        group(g + 3, std::integral_constant<int, 3>{});
    }
    // The last K groups issued loads for groups past the end (zero-size resources) that nothing
    // waits for: B registers, zero-points, scales and stage DMA. Their data may land at any time
    // until they complete, so every one of them completes here, and the registers they write stay
    // reserved up to this wait (the empty asm statements below read them): otherwise the epilogue
    // could reuse such a register for an address and have it overwritten by a late zero.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (kPacked) asm volatile("" : "+v"(rb[0]), "+v"(rb[1]));
    if constexpr (kHasZ) asm volatile("" : "+v"(zq));
    if constexpr (EPI == Epi::GroupScale) asm volatile("" : "+v"(sq));
    wait_sc(I0{}, I0{});
    wait_sc(I0{}, I1{});
#undef MQ_WAIT_B
    // drain: the last LAG tiles of the last group run (dead unless G is a multiple of four)
#pragma unroll
    for (int t = 0; t < LAG; ++t) {
        const int tp = NTL - LAG + t;
        if constexpr (EPI == Epi::GroupScale) fma_tile(tp, 1);
        if constexpr (EPI == Epi::GroupPartials)
            if (g1 - 1 < G) write_partials(tp, g1 - 1, true);
    }

    if constexpr (EPI == Epi::GroupPartials) return;


    if constexpr (EPI == Epi::RowAcc) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int64_t col = n0 + wn * WC + j * 16 + fr;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm * WR + i * 16 + 4 * (lane >> 4) + r;
                    if (row < M) a.part[row * N + col] = acci[i][j][r];
                }
            }
        return;
    }

    // ---- output epilogue: scale, bias, rounding to the output type; 16-bit types are staged through
    // LDS for 16-byte row stores
    __syncthreads();   // every wave is done with the pipeline stages the staging area reuses
    if constexpr (EPI == Epi::GroupScale) {
        const float cs_row = cs + __shfl_xor(cs, 1, 64);   // the two threads of the row
        if (bpart == 0 && (TN == TM || brow < TN)) lds<float>(smem, C_LDS + 4 * brow) = cs_row * kMagic;
        __syncthreads();
    }
    if constexpr (SPLIT) {
        // partial outputs of this K slice: fp32 sum_g s P (offset removed) or the int32 sum
        const int64_t slice_off = static_cast<int64_t>(slice) * M * N;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int lc = wn * WC + j * 16 + fr;
            const int64_t col = n0 + lc;
            if (col >= N) continue;
            float cv = 0.0f;
            if constexpr (EPI == Epi::GroupScale) cv = lds<float>(smem, C_LDS + 4 * lc);
#pragma unroll
            for (int i = 0; i < NI; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm * WR + i * 16 + 4 * (lane >> 4) + r;
                    if (row >= M) continue;
                    if constexpr (EPI == Epi::GroupScale)
                        static_cast<float*>(a.work)[slice_off + row * N + col] = (acc[i][j][r] - cv) * kSfacA;
                    else
                        static_cast<int32_t*>(a.work)[slice_off + row * N + col] = acci[i][j][r];
                }
        }
        return;
    }
    // column inputs of this lane (the fp32 weight scale or offset correction, the bias) and row
    // scales, all from LDS; rows and columns past the matrix read 0 and are never stored
    float colv[NJ], biasv[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int lc = wn * WC + j * 16 + fr;
        colv[j] = lds<float>(smem, C_LDS + 4 * lc);
        biasv[j] = lds<float>(smem, BI_LDS + 4 * lc);
    }
    // the row scales of rows 4 (lane / 16) + 0..3 of row block i
    auto row_scales = [&](int i) { return lds<f4>(smem, R_LDS + 4 * (wm * WR + i * 16 + 4 * (lane >> 4))); };
    // y[m, n] in fp32 before the rounding to the output type
    auto out_value = [&](int i, int j, int r, float sa_r) {
        if constexpr (EPI == Epi::GroupScale) return __builtin_fmaf(acc[i][j][r] - colv[j], sa_r, biasv[j]);
        else return static_cast<float>(acci[i][j][r]) * sa_r * colv[j] + biasv[j];
    };
    const bool full = m0 + TM <= M && n0 + TN <= N;   // no row or column of the tile past the matrix
    if (a.y_dtype == kDtF32) {
        // fp32 outputs straight from the registers: the 16 lanes of a row segment write 64
        // consecutive bytes
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const f4 sav = row_scales(i);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = m0 + wm * WR + i * 16 + 4 * (lane >> 4) + r;
                if (!full && row >= M) continue;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int64_t col = n0 + wn * WC + j * 16 + fr;
                    if (full || col < N) static_cast<float*>(a.y)[row * a.ldy + col] = out_value(i, j, r, sav[r]);
                }
            }
        }
        return;
    }
    uint16_t* stage = reinterpret_cast<uint16_t*>(smem) + wave * WR * OROW;
    // the staging loop once per 16-bit output type (a wave-uniform branch outside the loop)
    auto stage_tile = [&](auto DTc) {
        constexpr int DT = decltype(DTc)::value;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int lr0 = i * 16 + 4 * (lane >> 4);
            const f4 sav = row_scales(i);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int lc = j * 16 + fr;
#pragma unroll
                for (int r = 0; r < 4; r += 2) {
                    const uint32_t hb = pack_16x2(out_value(i, j, r, sav[r]), out_value(i, j, r + 1, sav[r + 1]), DT);
                    stage[(lr0 + r) * OROW + lc] = static_cast<uint16_t>(hb & 0xffffu);
                    stage[(lr0 + r + 1) * OROW + lc] = static_cast<uint16_t>(hb >> 16);
                }
            }
        }
    };
    if (a.y_dtype == kDtF16) stage_tile(std::integral_constant<int, kDtF16>{});
    else stage_tile(std::integral_constant<int, kDtBf16>{});
    __syncthreads();
    const int64_t col0 = n0 + wn * WC;
    // 16-byte row stores: a staged row holds 2 NJ chunks of 16 bytes; lane l of iteration it
    // writes chunk (64 it + l) % (2 NJ) of staged row (64 it + l) / (2 NJ)
    constexpr int kChunks = 2 * NJ, kStoreIt = WR * kChunks / 64;
    if (full && (a.ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) {
        uint16_t* ybase = static_cast<uint16_t*>(a.y) + (m0 + wm * WR) * a.ldy + col0;
#pragma unroll 4
        for (int it = 0; it < kStoreIt; ++it) {
            const int c = it * 64 + lane;
            const int lr = c / kChunks, ch = c % kChunks;
            *reinterpret_cast<uint4*>(ybase + lr * a.ldy + ch * 8) =
                *reinterpret_cast<const uint4*>(&stage[lr * OROW + ch * 8]);
        }
        return;
    }
#pragma unroll 4
    for (int it = 0; it < kStoreIt; ++it) {
        const int c = it * 64 + lane;
        const int lr = c / kChunks, ch = c % kChunks;
        const int64_t row = m0 + wm * WR + lr;
        const int64_t col = col0 + ch * 8;
        if (row >= M || col >= N) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(&stage[lr * OROW + ch * 8]);
        uint16_t* dst = static_cast<uint16_t*>(a.y) + row * a.ldy + col;
        if ((a.ldy % 8) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && col + 8 <= N) {
            *reinterpret_cast<uint4*>(dst) = v;
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (col + e < N) dst[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

// y[m, n] = T(sum_s part[s][m][n] * sa[m] + bias[n]) (GroupScale: fp32 partials) or
// T(float(sum_s part[s][m][n]) * sa[m] * ws[n] + bias[n]) (RowScale: int32 partials, the
// non-split epilogue's arithmetic on the exact full-K sum). 8 consecutive columns per thread.
template <bool INT>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs a) {
    const int64_t M = a.M, N = a.N;
    const int64_t cols8 = (N + 7) / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= M * cols8) return;
    const int64_t row = idx / cols8, col0 = (idx % cols8) * 8;
    const bool full = col0 + 8 <= N && N % 4 == 0;   // two aligned 16-byte loads per slice
    float t[8];
    if constexpr (INT) {
        int32_t sum[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int s = 0; s < a.ksplit; ++s) {
            const int32_t* p = static_cast<const int32_t*>(a.work) + (s * M + row) * N + col0;
            if (full) {
                const int4 u = *reinterpret_cast<const int4*>(p), v = *reinterpret_cast<const int4*>(p + 4);
                sum[0] += u.x; sum[1] += u.y; sum[2] += u.z; sum[3] += u.w;
                sum[4] += v.x; sum[5] += v.y; sum[6] += v.z; sum[7] += v.w;
            } else {
                for (int e = 0; e < 8 && col0 + e < N; ++e) sum[e] += p[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = static_cast<float>(sum[e]) * a.sa[row] * (col0 + e < N ? a.ws32[col0 + e] : 0.0f);
    } else {
        float sum[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        for (int s = 0; s < a.ksplit; ++s) {
            const float* p = static_cast<const float*>(a.work) + (s * M + row) * N + col0;
            if (full) {
                const float4 u = *reinterpret_cast<const float4*>(p), v = *reinterpret_cast<const float4*>(p + 4);
                sum[0] += u.x; sum[1] += u.y; sum[2] += u.z; sum[3] += u.w;
                sum[4] += v.x; sum[5] += v.y; sum[6] += v.z; sum[7] += v.w;
            } else {
                for (int e = 0; e < 8 && col0 + e < N; ++e) sum[e] += p[e];
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) t[e] = sum[e] * a.sa[row];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
        if (a.bias && col0 + e < N) t[e] += load_as_f32(a.bias, a.bias_dtype, col0 + e);
    const bool vec = col0 + 8 <= N;
    if (a.y_dtype == kDtF32) {
        float* dst = static_cast<float*>(a.y) + row * a.ldy + col0;
        if (vec && a.ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) {
            *reinterpret_cast<float4*>(dst) = float4{t[0], t[1], t[2], t[3]};
            *reinterpret_cast<float4*>(dst + 4) = float4{t[4], t[5], t[6], t[7]};
        } else {
            for (int e = 0; e < 8 && col0 + e < N; ++e) dst[e] = t[e];
        }
        return;
    }
    uint32_t out[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = pack_16x2(t[2 * e], t[2 * e + 1], a.y_dtype);
    uint16_t* dst = static_cast<uint16_t*>(a.y) + row * a.ldy + col0;
    if (vec && a.ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0) {
        *reinterpret_cast<uint4*>(dst) = uint4{out[0], out[1], out[2], out[3]};
    } else {
        for (int e = 0; e < 8 && col0 + e < N; ++e) dst[e] = static_cast<uint16_t>(out[e >> 1] >> (16 * (e & 1)));
    }
}

template <int TM, int TN, WKind WK, Epi EPI, int AM, bool XP>
int launch_tile(const GemmArgs& a, hipStream_t stream) {
    const int tiles_m = static_cast<int>((a.M + TM - 1) / TM);
    const int tiles_n = static_cast<int>((a.N + TN - 1) / TN);
    if constexpr (EPI == Epi::GroupScale || EPI == Epi::RowScale) {
        if (a.ksplit > 1) {
            hipLaunchKernelGGL((gemm_wide_kernel<TM, TN, WK, EPI, AM, true, XP>),
                               dim3(static_cast<unsigned>(tiles_m * tiles_n * a.ksplit)), dim3(NT), 0, stream, a,
                               tiles_m, tiles_n);
            const int rc = launch_status("gemm_wide");
            if (rc) return rc;
            const int64_t threads = a.M * ((a.N + 7) / 8);
            hipLaunchKernelGGL(splitk_reduce_kernel<EPI == Epi::RowScale>, dim3(static_cast<unsigned>((threads + 255) / 256)),
                               dim3(256), 0, stream, a);
            return launch_status("gemm_splitk_reduce");
        }
    }
    hipLaunchKernelGGL((gemm_wide_kernel<TM, TN, WK, EPI, AM, false, XP>), dim3(static_cast<unsigned>(tiles_m * tiles_n)),
                       dim3(NT), 0, stream, a, tiles_m, tiles_n);
    return launch_status("gemm_wide");
}

template <WKind WK, Epi EPI, int AM, bool XP = false>
int launch_one(const GemmArgs& a, hipStream_t stream) {
    const int t = a.tile ? a.tile : choose_tile(a.M, a.N);
    if (t == 128) return launch_tile<128, 128, WK, EPI, AM, XP>(a, stream);
    if (t == 192) return launch_tile<256, 192, WK, EPI, AM, XP>(a, stream);
    if (t == 256) return launch_tile<256, 256, WK, EPI, AM, XP>(a, stream);
    set_error("gemm: tile code %d is not 128, 192 or 256", t);
    return -1;
}

template <WKind WK, Epi EPI, bool XP = false>
int launch_group(const GemmArgs& a, hipStream_t stream) {
    switch (a.act_mode) {
        case 0: return launch_one<WK, EPI, 0, XP>(a, stream);
        case 2: return launch_one<WK, EPI, 2, XP>(a, stream);
        default: break;
    }
    set_error("gemm: unknown activation layout %d", a.act_mode);
    return -1;
}

template <WKind WK>
int launch_wk(const GemmArgs& a, Epi epi, hipStream_t stream) {
    if constexpr (WK != WKind::I8) {   // 4-bit weights: per-group scales
        if (a.wtile) {                  // expanded to int8 tiles
            if (epi == Epi::GroupScale) return launch_group<WK, Epi::GroupScale, true>(a, stream);
            set_error("gemm: expanded 4-bit weights serve the group-scale epilogue only");
            return -2;
        }
        if (epi == Epi::GroupScale) return launch_group<WK, Epi::GroupScale>(a, stream);
        if (epi == Epi::GroupPartials) return launch_group<WK, Epi::GroupPartials>(a, stream);
    }
    if constexpr (WK != WKind::U4Asym) {   // full-K accumulators: signed int4 or int8 weights
        if (epi == Epi::RowScale) return launch_one<WK, Epi::RowScale, 0>(a, stream);
        if (epi == Epi::RowAcc) return launch_one<WK, Epi::RowAcc, 0>(a, stream);
    }
    set_error("gemm: unsupported weight kind / epilogue combination");
    return -2;
}

}  // namespace

int choose_tile(int64_t M, int64_t N) {
    const int cus = device_cu_count();
    if (cus <= 0) return 256;
    const int64_t tm = (M + 255) / 256, tiles256 = tm * ((N + 255) / 256), tiles192 = tm * ((N + 191) / 192);
    if (2 * tiles256 <= cus) return 128;
    // Rounds of resident workgroups, in tenths of a 256 x 256 round. A 256 x 192 round costs 0.9 (3/4
    // of the MFMAs but the same loads, unpack and LDS traffic per K group: measured 0.87-0.97 of a
    // 256 x 256 round). A last 256 x 256 round of
    // whole tile rows on at most a quarter of the compute units runs as its own product on smaller
    // tiles (tail_rows), costed 0.3.
    const int64_t tn = (N + 255) / 256, full = tiles256 / cus, part = tiles256 % cus;
    const bool tail = full > 0 && part > 0 && part % tn == 0 && 4 * part <= cus;
    const int64_t c256 = 10 * full + (part == 0 ? 0 : tail ? 3 : 10);
    const int64_t c192 = 9 * ((tiles192 + cus - 1) / cus);
    return c192 < c256 ? 192 : 256;
}

int choose_ksplit(int64_t M, int64_t N, int64_t K, int64_t work_bytes, int* kgroups, bool int_sums) {
    *kgroups = 0;
    if (M <= 128 || K < 192 || K % TK) return 1;               // the few-row kernels have no split
    const int cus = device_cu_count();
    if (cus <= 0) return 1;
    const int t = choose_tile(M, N), tr = tile_rows(t);
    const int64_t tiles = ((M + tr - 1) / tr) * ((N + t - 1) / t);
    const int64_t blocks = (K / TK + 3) / 4;                    // blocks of four K groups
    // int32 row-scale sums (no per-group fmas) are quick per K group: their partial outputs pay
    // for themselves only over a long K
    if (2 * tiles > cus || blocks < (int_sums ? 16 : 4)) return 1;
    // at least two blocks per slice; as many slices as give every compute unit a workgroup
    int64_t s = std::min<int64_t>(cus / tiles, blocks / 2);
    const int64_t per = (blocks + s - 1) / s;                   // blocks per slice
    s = (blocks + per - 1) / per;
    if (s < 2 || s * M * N * 4 > work_bytes) return 1;
    *kgroups = static_cast<int>(per * 4);
    return static_cast<int>(s);
}

int64_t tail_rows(int64_t M, int64_t N, int64_t K) {
    constexpr int64_t T = 256;   // only products on 256 tiles leave such a last wave
    if (M <= T || K % TK || choose_tile(M, N) != T) return 0;
    const int cus = device_cu_count();
    if (cus <= 0) return 0;
    const int64_t tiles_m = (M + T - 1) / T, tiles_n = (N + T - 1) / T;
    const int64_t r = (tiles_m * tiles_n) % cus;   // tiles of the last, partial wave
    if (tiles_m * tiles_n <= cus || r == 0 || r % tiles_n || 4 * r > cus) return 0;
    return M - (tiles_m - r / tiles_n) * T;
}

int64_t workspace_bytes(int64_t M, int64_t N, int64_t K, bool int_sums) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    int kgroups = 0;
    const int64_t tail = tail_rows(M, N, K);
    const int64_t rows = tail > 0 ? tail : M;
    const int s = choose_ksplit(rows, N, K, INT64_MAX, &kgroups, int_sums);
    return s > 1 ? static_cast<int64_t>(s) * rows * N * 4 : 0;
}

int launch_gemm_wide(const GemmArgs& a, WKind wk, Epi epi, hipStream_t stream) {
    switch (wk) {
        case WKind::U4Asym: return launch_wk<WKind::U4Asym>(a, epi, stream);
        case WKind::I4Sym: return launch_wk<WKind::I4Sym>(a, epi, stream);
        case WKind::I8: return launch_wk<WKind::I8>(a, epi, stream);
    }
    set_error("gemm: unsupported weight kind / epilogue combination");
    return -2;
}

}  // namespace mq
