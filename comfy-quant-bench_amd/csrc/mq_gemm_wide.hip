// Large-tile quantized GEMM for gfx950: 256 x 256 output tile per workgroup of 8 wavefronts,
// int8 MFMA (v_mfma_i32_16x16x64_i8: one instruction covers one 64-wide K group of a 16 x 16
// output tile), one K group per k-step.
//
// Layout. Waves form a 4 (M) x 2 (N) grid; each owns a 64 x 128 output tile made of 4 x 8 MFMA
// 16x16 tiles. In the 16x16 output layout lane l holds column l % 16 and rows 4 * (l / 16) + r,
// r = 0..3, so every lane needs one weight scale per column tile. A (int8 activation codes) and
// B (weights, unpacked to int8 on their way into LDS) are double-buffered in LDS as 64-byte rows
// whose four 16-byte chunks are XOR-swizzled by (row >> 1) & 3: the fragment reads (lane l reads
// chunk l / 16 of row l % 16) are then free of bank conflicts on gfx950, which a padded pitch of 80
// bytes is not (measured). Global loads run two K groups ahead of the group being multiplied, in
// two register sets.
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
// bytes at a time: lo/hi nibble masks, ((v | 0x80) - z) ^ 0x80 per byte (no inter-byte borrow) for
// q - z, ((z | 0x80) - v) ^ 0x80 for z - q, and two byte permutes back to k order. Signed int4
// is the same with v ^ 8 and z = 8.
//
// int4 activations. With codes in [-7, 7] the partials are ~100x smaller than with int8 codes and
// the fp32 step above would lose accuracy, so int4 operands are scaled by 16 (exact in int8):
// activation layout 1 scales them on their way into LDS; layout 2 (written by the rotate+quantize
// kernel) stores 16 * q negated in odd groups, and signed int4 weights then enter as 16 * v. The
// MFMA result is 2^gshift times the partial (gshift 4 or 8) and the scales are divided by the same
// power of two, so every step stays exact.
#include <type_traits>

#include "mq_device.h"
#include "mq_internal.h"

namespace mq {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

constexpr int TM = 256, TN = 256, TK = 64;
constexpr int NT = 512;                   // threads per workgroup
constexpr int LROW = 64;                  // LDS pitch of A / B tile rows (bytes)
constexpr int OROW = 136;                 // bf16 pitch of the output staging rows (128 + 8)
constexpr int kSeed = 0x4B400000;         // bits of 1.5 * 2^23

constexpr int NSTAGE = 3;                 // LDS ring of K groups
struct alignas(16) Pipe {
    alignas(16) int8_t a[NSTAGE][TM * LROW];
    alignas(16) int8_t b[NSTAGE][TN * LROW];
    alignas(16) float s[NSTAGE][TN];
};
struct alignas(16) Smem {
    union alignas(16) {
        Pipe pipe;
        alignas(16) uint16_t out[8][64 * OROW];
    } u;
    alignas(16) float corr[TN];
};

__device__ __forceinline__ void unpack_pos(uint32_t w, uint32_t zz, uint32_t& o0, uint32_t& o1) {
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    lo = ((lo | 0x80808080u) - zz) ^ 0x80808080u;
    hi = ((hi | 0x80808080u) - zz) ^ 0x80808080u;
    o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

__device__ __forceinline__ void unpack_neg(uint32_t w, uint32_t zz80, uint32_t& o0, uint32_t& o1) {
    uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
    lo = (zz80 - lo) ^ 0x80808080u;
    hi = (zz80 - hi) ^ 0x80808080u;
    o0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
    o1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
}

// 32 packed 4-bit weights (16 bytes, one half of a row's K group) -> 32 int8 operands in k order.
// U4Asym: q - z (z - q when NEG); I4Sym: v (-v when NEG), or 16 * v when X16 (never negated).
template <WKind WK, bool NEG, bool X16>
__device__ __forceinline__ void unpack_weights(uint4 w, uint32_t zb, uint4& u0, uint4& u1) {
    if constexpr (WK == WKind::I4Sym && X16) {
        const uint32_t in[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // a nibble moved to the high half of its byte reads as 16 x its signed value
            const uint32_t lo = (in[e] << 4) & 0xf0f0f0f0u, hi = in[e] & 0xf0f0f0f0u;
            o[2 * e] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
            o[2 * e + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
        }
        u0 = make_uint4(o[0], o[1], o[2], o[3]);
        u1 = make_uint4(o[4], o[5], o[6], o[7]);
    } else {
        if constexpr (WK == WKind::I4Sym) {
            // signed nibble v -> v ^ 8 in [0, 15] with zero-point 8 (a zero-filled row stays 0)
            w.x ^= 0x88888888u; w.y ^= 0x88888888u; w.z ^= 0x88888888u; w.w ^= 0x88888888u;
            zb = 8u;
        }
        const uint32_t zz = zb * 0x01010101u;
        if constexpr (NEG) {
            const uint32_t zz80 = zz | 0x80808080u;
            unpack_neg(w.x, zz80, u0.x, u0.y);
            unpack_neg(w.y, zz80, u0.z, u0.w);
            unpack_neg(w.z, zz80, u1.x, u1.y);
            unpack_neg(w.w, zz80, u1.z, u1.w);
        } else {
            unpack_pos(w.x, zz, u0.x, u0.y);
            unpack_pos(w.y, zz, u0.z, u0.w);
            unpack_pos(w.z, zz, u1.x, u1.y);
            unpack_pos(w.w, zz, u1.z, u1.w);
        }
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

// Buffer resource over [base, base + bytes): loads outside the range return 0. Invalid rows are
// given the offset kOob, which is out of range whatever the scalar offset adds to it.
constexpr int kOob = static_cast<int>(0x80000000u);
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                            static_cast<int>(bytes), 0x00020000);
}
__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Global loads of K group g into registers (A: two 16-byte chunks; B: one packed or two int8
// chunks; the zero-point byte and fp16 scale of this thread's weight row).
template <WKind WK, Epi EPI>
__device__ __forceinline__ void gload_group(int g, __amdgpu_buffer_rsrc_t ra_rs, __amdgpu_buffer_rsrc_t rb_rs,
                                            __amdgpu_buffer_rsrc_t rz_rs, __amdgpu_buffer_rsrc_t rs_rs,
                                            const int (&a_off)[2], const int (&b8_off)[2], int b_off, int z_off,
                                            int s_off, uint4 (&ra)[2], uint4 (&rb)[2], uint32_t& rz, uint32_t& rs) {
#pragma unroll
    for (int c = 0; c < 2; ++c) ra[c] = ld128(ra_rs, a_off[c], g * TK);
    if constexpr (WK != WKind::I8) {
        rb[0] = ld128(rb_rs, b_off, g * (TK / 2));
    } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) rb[c] = ld128(rb_rs, b8_off[c], g * TK);
    }
    if constexpr (WK == WKind::U4Asym) rz = __builtin_amdgcn_raw_buffer_load_b8(rz_rs, z_off, g >> 1, 0);
    if constexpr (EPI == Epi::GroupScale) rs = __builtin_amdgcn_raw_buffer_load_b16(rs_rs, s_off, 2 * g, 0);
}

// One workgroup: a 256 x 256 output tile. AM is the activation layout of the group epilogues
// (0 int8 codes; 1 int4 codes, scaled by 16 on their way into LDS; 2 int4 codes stored as 16 * q
// and negated in odd groups, signed int4 weights then entering as 16 * v); row epilogues use 0.
template <WKind WK, Epi EPI, int AM>
__global__ void __launch_bounds__(NT) gemm_wide_kernel(GemmArgs a, int tiles_m, int tiles_n) {
    constexpr bool kGroup = EPI == Epi::GroupScale || EPI == Epi::GroupPartials;
    constexpr bool kPacked = WK != WKind::I8;
    constexpr int kShift = kGroup ? (AM == 1 ? 4 : AM == 2 ? (WK == WKind::I4Sym ? 8 : 4) : 0) : 0;
    __shared__ Smem sm;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    map_tile(static_cast<int>(blockIdx.x), tiles_m, tiles_n, tm, tn);
    const int64_t m0 = static_cast<int64_t>(tm) * TM, n0 = static_cast<int64_t>(tn) * TN;
    const int64_t M = a.M, N = a.N;
    const int G = static_cast<int>(a.K / TK);
    const int rows_m = M - m0 < TM ? static_cast<int>(M - m0) : TM;   // valid rows of this tile
    const int rows_n = N - n0 < TN ? static_cast<int>(N - n0) : TN;
    const int kbytes_w = kPacked ? static_cast<int>(a.K / 2) : static_cast<int>(a.K);

    // ---- loader roles. A (and I8 B): chunks tid and tid + 512 of 16 bytes, 4 per 64-byte row.
    const int lrow = tid >> 2, lpart = tid & 3;
    const int brow = tid >> 1, bhalf = tid & 1;   // packed B: 2 threads per weight row
    const auto ra_rs = rsrc(a.qa + m0 * a.lda, (rows_m - 1) * a.lda + a.K);
    const auto rb_rs = rsrc(a.qw + n0 * a.ldw, (rows_n - 1) * a.ldw + kbytes_w);
    int a_off[2], b8_off[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int r = lrow + 128 * c;
        a_off[c] = r < rows_m ? static_cast<int>(r * a.lda) + lpart * 16 : kOob;
        b8_off[c] = r < rows_n ? static_cast<int>(r * a.ldw) + lpart * 16 : kOob;
    }
    const bool b_ok = brow < rows_n;
    const int b_off = b_ok ? static_cast<int>(brow * a.ldw) + bhalf * 16 : kOob;
    // zero-points and scales (null for the kinds that have none: the range is then empty)
    const bool has_z = WK == WKind::U4Asym, has_s = EPI == Epi::GroupScale;
    const auto rz_rs = rsrc(has_z ? a.wz + n0 * a.ldwz : a.qw, has_z ? (rows_n - 1) * a.ldwz + (G + 1) / 2 : 0);
    const auto rs_rs = rsrc(has_s ? a.ws16 + n0 * a.ldws : reinterpret_cast<const uint16_t*>(a.qw),
                            has_s ? ((rows_n - 1) * a.ldws + G) * 2 : 0);
    const int z_off = has_z && b_ok ? static_cast<int>(brow * a.ldwz) : kOob;
    const int s_off = has_s && b_ok ? static_cast<int>(brow * a.ldws * 2) : kOob;

    // one register set carries a K group from its global load to its LDS store
    uint4 ra[2], rb[2];
    uint32_t rz = 0, rs = 0;
#define MQ_GLOAD(g) gload_group<WK, EPI>(g, ra_rs, rb_rs, rz_rs, rs_rs, a_off, b8_off, b_off, z_off, s_off, ra, rb, rz, rs)
    constexpr float kSfac = 1.0f / static_cast<float>(1 << kShift);
    float cs = 0.0f;   // sum_g (-1)^g s[n, g] for this thread's weight row (GroupScale)
    // byte offset of 16-byte chunk c of tile row r in the swizzled LDS layout
    auto lds_off = [](int r, int c) { return r * LROW + ((c ^ ((r >> 1) & 3)) << 4); };
    // Store the register set (group g_data, or a repeat of the last group past the end) into
    // stage `stage`; NEG is the parity of the group the stage is for. `real` says whether that
    // group exists (its scale then enters the offset sum).
    auto lstore = [&](int stage, auto NEGC, bool real) {
        constexpr bool neg = kGroup && decltype(NEGC)::value;
        constexpr bool neg_w = neg && AM != 2;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            uint4 v = ra[c];
            if constexpr (AM == 1 && kGroup)
                v = make_uint4((v.x << 4) & 0xf0f0f0f0u, (v.y << 4) & 0xf0f0f0f0u, (v.z << 4) & 0xf0f0f0f0u,
                               (v.w << 4) & 0xf0f0f0f0u);
            *reinterpret_cast<uint4*>(&sm.u.pipe.a[stage][lds_off(lrow + 128 * c, lpart)]) = v;
        }
        if constexpr (kPacked) {
            uint4 u0, u1;
            const uint32_t zb = (rz >> (neg ? 4 : 0)) & 0xfu;
            unpack_weights<WK, neg_w, AM == 2 && kGroup>(rb[0], zb, u0, u1);
            *reinterpret_cast<uint4*>(&sm.u.pipe.b[stage][lds_off(brow, 2 * bhalf)]) = u0;
            *reinterpret_cast<uint4*>(&sm.u.pipe.b[stage][lds_off(brow, 2 * bhalf + 1)]) = u1;
        } else {
#pragma unroll
            for (int c = 0; c < 2; ++c)
                *reinterpret_cast<uint4*>(&sm.u.pipe.b[stage][lds_off(lrow + 128 * c, lpart)]) = rb[c];
        }
        if constexpr (EPI == Epi::GroupScale) {
            // both threads of a row store the same value (no divergent branch)
            float sv = f16_bits_to_f32(static_cast<uint16_t>(rs)) * kSfac;   // exact: power of two
            sv = neg ? -sv : sv;
            sm.u.pipe.s[stage][brow] = sv;
            cs += real ? sv : 0.0f;
        }
    };

    // fragment reads: lane l reads chunk l / 16 of row l % 16 of a 16-row block (swizzle depends
    // only on the row within the block, so one per-lane offset serves every block)
    const int fr = lane & 15, fk = ((lane >> 4) ^ ((fr >> 1) & 3)) << 4;
    const int a_frag = (wm * 64 + fr) * LROW + fk;    // + i * 16 * LROW
    const int b_frag = (wn * 128 + fr) * LROW + fk;   // + j * 16 * LROW
    const int s_frag = wn * 128 + fr;                 // + j * 16
    const v4i seed = {kSeed, kSeed, kSeed, kSeed};

    float acc[4][8][4];
    v4i acci[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[i][j][r] = 0.0f;
                acci[i][j][r] = 0;
            }
        }

    // Fragment registers: A of the current K group (fragment i is refilled with group g + 1's
    // right after its last MFMA in group g), and a 4-slot ring of B fragments and scales (slot =
    // column % 4, 8 columns per group) read two columns ahead; the last two columns of group g
    // fetch columns 0 and 1 of group g + 1.
    v4i fa[4], fb[4];
    float fs[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto read_a = [&](int stage, int i, v4i& dst) {
        dst = *reinterpret_cast<const v4i*>(&sm.u.pipe.a[stage][a_frag + i * 16 * LROW]);
    };
    auto read_b = [&](int stage, int j, v4i& dst, float& sdst) {
        dst = *reinterpret_cast<const v4i*>(&sm.u.pipe.b[stage][b_frag + j * 16 * LROW]);
        if constexpr (EPI == Epi::GroupScale) sdst = sm.u.pipe.s[stage][s_frag + j * 16];
    };
    using T0 = std::integral_constant<int, 0>;
    using T1 = std::integral_constant<int, 1>;

    // prologue: groups 0 and 1 into LDS stages 0 and 1, group 2 in registers (group indices are
    // clamped to the last group: the repeats are never read)
    const int glast = G - 1;
    MQ_GLOAD(0);
    lstore(0, T0{}, true);
    MQ_GLOAD(1 < glast ? 1 : glast);
    lstore(1, T1{}, G > 1);
    MQ_GLOAD(2 < glast ? 2 : glast);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i) read_a(0, i, fa[i]);
    read_b(0, 0, fb[0], fs[0]);
    read_b(0, 1, fb[1], fs[1]);

    // K group g: 32 MFMA tiles t = 4 j + i, column-major. Every step issues tile t's MFMA, then the
    // fmas of tile t - 1 (MFMA and VALU work overlap, two tiles of results are live); a scheduling
    // fence after each step keeps every LDS read and store where it is written, so the reads really
    // run two columns ahead. After column 1 the stage of group g + 2 is filled from the register
    // set and the global loads of group g + 3 are issued. One barrier per group: stage
    // (g + 2) % 3 was last read before the previous barrier, group g + 1's stage was completed
    // before it. The body is branch-free: past the last group, loads and stores repeat the last
    // group (never read), so each group is one scheduling region.
    auto step = [&](int g, auto P) {
        constexpr int par = decltype(P)::value;   // g & 1
        const int st = g % NSTAGE, st1 = (g + 1) % NSTAGE, st2 = (g + 2) % NSTAGE;
        constexpr int LAG = 1;   // tile t's fmas run LAG steps after its MFMA
        v4i d[LAG + 1];
        v4i seedv = seed;
#pragma unroll
        for (int t = 0; t < 32 + LAG; ++t) {
            if (t < 32) {
                const int j = t >> 2, i = t & 3;
                if (i == 0) {
                    // two columns ahead, into the slot of column j - 2 (its MFMAs and fmas are done)
                    const int jj = j + 2;
                    if (jj < 8) read_b(st, jj, fb[jj & 3], fs[jj & 3]);
                    else read_b(st1, jj - 8, fb[jj & 3], fs[jj & 3]);
                }
                if (t == 8) {
                    lstore(st2, std::integral_constant<int, par>{}, g + 2 < G);
                    MQ_GLOAD(g + 3 < glast ? g + 3 : glast);
                }
                // empty asm on the seed: the MFMA cannot be hoisted above this step
                asm volatile("" : "+v"(seedv));
                if constexpr (kGroup) {
                    d[t % (LAG + 1)] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j & 3], seedv, 0, 0, 0);
                    if constexpr (EPI == Epi::GroupPartials) {
                        const int64_t col = n0 + wn * 128 + j * 16 + fr;
                        int32_t* part = a.part + static_cast<int64_t>(g) * M * N;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int64_t row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                            const int32_t pv = (d[t % (LAG + 1)][r] - kSeed) >> kShift;   // exact: a multiple of 2^kShift
                            if (row < M && col < N) part[row * N + col] = par ? -pv : pv;
                        }
                    }
                } else {
                    acci[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j & 3], acci[i][j], 0, 0, 0);
                }
                if (j == 7) read_a(st1, i, fa[i]);   // fa[i]'s last use in group g
            }
            if constexpr (EPI == Epi::GroupScale) {
                if (t >= LAG) {
                    const int tp = t - LAG, jp = tp >> 2, ip = tp & 3;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[ip][jp][r] = __builtin_fmaf(__int_as_float(d[tp % (LAG + 1)][r]), fs[jp & 3], acc[ip][jp][r]);
                    // empty asm on the accumulators: the fmas complete in this step (not sunk)
                    asm volatile("" : "+v"(acc[ip][jp][0]), "+v"(acc[ip][jp][1]), "+v"(acc[ip][jp][2]),
                                 "+v"(acc[ip][jp][3]));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        __syncthreads();
    };
    for (int g = 0; g < G; g += 2) {
        step(g, T0{});
        if (g + 1 < G) step(g + 1, T1{});
    }
#undef MQ_GLOAD

    if constexpr (EPI == Epi::GroupPartials) return;

    if constexpr (EPI == Epi::RowAcc) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int64_t col = n0 + wn * 128 + j * 16 + fr;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t row = m0 + wm * 64 + i * 16 + 4 * (lane >> 4) + r;
                    if (row < M) a.part[row * N + col] = acci[i][j][r];
                }
            }
        return;
    }

    // ---- output epilogue: scale, bias, bf16, staged through LDS for 16-byte row stores
    if constexpr (EPI == Epi::GroupScale) {
        if (bhalf == 0) sm.corr[brow] = cs * kMagic;
        __syncthreads();
    }
    float colv[8], biasv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const int lc = wn * 128 + j * 16 + fr;
        const int64_t col = n0 + lc;
        const bool ok = col < N;
        if constexpr (EPI == Epi::GroupScale) colv[j] = sm.corr[lc];
        else colv[j] = ok ? a.ws32[col] : 0.0f;
        biasv[j] = (ok && a.bias) ? __uint_as_float(static_cast<uint32_t>(a.bias[col]) << 16) : 0.0f;
    }
    uint16_t* stage = sm.u.out[wave];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int lr0 = i * 16 + 4 * (lane >> 4);
        const int64_t row0 = m0 + wm * 64 + lr0;
        float sav[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sav[r] = row0 + r < M ? a.sa[row0 + r] : 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int lc = j * 16 + fr;
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                f2 v;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    float t;
                    if constexpr (EPI == Epi::GroupScale)
                        t = (acc[i][j][r + e] - colv[j]) * sav[r + e] + biasv[j];
                    else
                        t = static_cast<float>(acci[i][j][r + e]) * sav[r + e] * colv[j] + biasv[j];
                    v[e] = t;
                }
                const bf2 h = __builtin_convertvector(v, bf2);
                const uint32_t hb = __builtin_bit_cast(uint32_t, h);
                stage[(lr0 + r) * OROW + lc] = static_cast<uint16_t>(hb & 0xffffu);
                stage[(lr0 + r + 1) * OROW + lc] = static_cast<uint16_t>(hb >> 16);
            }
        }
    }
    __syncthreads();
    const int64_t col0 = n0 + wn * 128;
    const bool vec_ok = (a.ldy % 8) == 0;
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
        const int c = it * 64 + lane;
        const int lr = c >> 4, ch = c & 15;
        const int64_t row = m0 + wm * 64 + lr;
        const int64_t col = col0 + ch * 8;
        if (row >= M || col >= N) continue;
        const uint4 v = *reinterpret_cast<const uint4*>(&stage[lr * OROW + ch * 8]);
        uint16_t* dst = a.y + row * a.ldy + col;
        if (vec_ok && col + 8 <= N) {
            *reinterpret_cast<uint4*>(dst) = v;
        } else {
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (col + e < N) dst[e] = static_cast<uint16_t>(w[e >> 1] >> (16 * (e & 1)));
        }
    }
}

template <WKind WK, Epi EPI, int AM>
int launch_one(const GemmArgs& a, hipStream_t stream) {
    const int tiles_m = static_cast<int>((a.M + TM - 1) / TM);
    const int tiles_n = static_cast<int>((a.N + TN - 1) / TN);
    hipLaunchKernelGGL((gemm_wide_kernel<WK, EPI, AM>), dim3(static_cast<unsigned>(tiles_m * tiles_n)), dim3(NT), 0,
                       stream, a, tiles_m, tiles_n);
    return launch_status("gemm_wide");
}

template <WKind WK, Epi EPI>
int launch_group(const GemmArgs& a, hipStream_t stream) {
    switch (a.act_mode) {
        case 0: return launch_one<WK, EPI, 0>(a, stream);
        case 1: return launch_one<WK, EPI, 1>(a, stream);
        case 2: return launch_one<WK, EPI, 2>(a, stream);
        default: break;
    }
    set_error("gemm: unknown activation layout %d", a.act_mode);
    return -1;
}

template <WKind WK>
int launch_wk(const GemmArgs& a, Epi epi, hipStream_t stream) {
    if constexpr (WK != WKind::I8) {   // 4-bit weights: per-group scales
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
