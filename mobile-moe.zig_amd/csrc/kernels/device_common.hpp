// Device-side building blocks shared by the gfx950 kernels.
//
// Tile layouts (built once at upload by codec.hip; same bytes per block as
// GGUF, only reordered):
//
//   A "row tile" is 16 consecutive output rows. For each row tile the kernels
//   read one 1 KiB record unit per 256 (IQ2_XXS) or 64 (Q8_0) input columns:
//   64 lanes x 16 B, one coalesced 128-bit load per lane. Lane l serves output
//   row n = l % 16 and column group g = l / 16 (8 consecutive columns of each
//   32-column block), which is the B-operand layout of
//   v_mfma_i32_16x16x32_i8 (B[k][n] with k = 8g..8g+7 in lane 16g+n).
//
//   IQ2_XXS unit (one 256-column superblock of 16 rows, 1056 B = 16 x 66 B):
//     recs: lane l holds 4 dwords; dword k covers sub-blocks 2k and 2k+1.
//     A record is the group's grid index idx and 7-bit sign code, split as
//     window = b012 | P<<3 | idx<<4 (12 bits) and hi3, where b012 = code
//     bits 0..2, hi3 = code bits 4..6 and P = parity(code bits 0..3):
//       bits  0.. 2  hi3 of sub-block 2k+1
//       bits  3..14  window of sub-block 2k
//       bits 15..17  hi3 of sub-block 2k
//       bits 18..29  window of sub-block 2k+1
//       bits 30..31  two bits of a sub-block scale ls (below)
//     Dwords 0,1 carry ls of sub-block g, dwords 2,3 ls of sub-block 4+g.
//     15 information bits per record + 8 ls bits per lane = the raw format's
//     64 bits per sub-block-row exactly.
//     d: 16 x f16, one per row.
//   Signed int8 weights: one 8-byte LDS table entry per record, addressed
//   straight from the dword (byte address d & 0x7FF8 for sub-block 2k,
//   (d >> 15) & 0x7FF8 for 2k+1), holds all eight weights with the signs of
//   b012, P (column 3: P ^ parity(b012)) and column 7 = P; the hi3 signs
//   (columns 4..6, and column 7 flipped by parity(hi3): the ksigns parity
//   bit) come from an 8-entry table of byte masks right after it, keyed by
//   hi3, and are applied with one xor-add (negate_bytes).
//
//   Q8_0 unit (two 32-column blocks of 16 rows, 1088 B = 32 x 34 B):
//     recs: lane l holds qs[8g..8g+7] of block 2u then of block 2u+1.
//     d:    16 x (f16 d(2u), f16 d(2u+1)).
//
// Activations are quantised per 32-column block to 16-bit fixed point split
// in two int8 digits (x ~= s * (256 * hi + lo)), so one int8 MFMA over a
// 32-column block yields exact integer partial sums for both digits.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace mmhip {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kTileRows = 16;
constexpr int kIq2UnitCols = 256;
constexpr int kQ8UnitCols = 64;
constexpr float kDigitMax = 32512.0f;  // 127 * 256: hi digit stays in [-127, 127]
constexpr int kIq2TableWords = 8192;   // 4096 record entries of two u32
constexpr int kIq2MaskWords = 16;      // hi3 sign masks (mask, mask & 0x01010101), after the record entries
constexpr int kIq2LdsWords = kIq2TableWords + kIq2MaskWords;
// LDS A layout (decode): per 256-column group, lane (m = 0|1, g) owns a
// 64-byte run holding the 8 A operands (8 x 8 digits) of the group's 8
// blocks for A row m (hi/lo digits) and column group g; runs are 80 B apart so
// the 8 lanes' 128-bit reads hit disjoint LDS banks.
constexpr int kARun = 80;
constexpr int kAGroupBytes = 8 * kARun;  // 640 B per 256 columns

// IEEE binary16 bits -> binary32, bit-exact (dequant.zig:19-47 semantics:
// subnormals normalised, Inf/NaN payload kept), independent of the device's
// f16 denormal mode: subnormals are m * 2^-24, computed exactly in f32.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-24f));
    uint32_t bits = (e == 31u) ? (s | 0x7F800000u | (m << 13)) : (s | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(bits);
}

// Hardware conversion for scales that only feed products: exact for every
// finite value (f16 denormals are enabled for these kernels); NaNs may come
// out quieted, which cannot change a product that is NaN anyway.
__device__ __forceinline__ float f16_scale(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// Workgroup barrier that orders LDS only. __syncthreads() is a workgroup-
// scope fence on all memory, which makes every wave wait for all of its
// outstanding global loads (the prefetched weight stream) at the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A wave-uniform value held in an SGPR from here on. Kernel arguments read
// through a runtime index (a launch's segment) are otherwise re-loaded where
// they are used, and each such scalar load inside a loop costs a wait on
// lgkmcnt, which also waits for the wave's outstanding LDS reads.
__device__ __forceinline__ uint32_t keep_sgpr(uint32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}

// Every field of a GEMV's arguments (GemvArgs) that a workgroup reads before
// its first weight load, read at once: the asm takes them all in SGPRs, so
// their scalar loads go out as one batch with one wait. Read where first
// used, each early-exit branch waited for its own loads: a chain of six
// kernel-argument round trips, about 1 us, before the first vector load.
template <class Args>
__device__ __forceinline__ void pin_gemv_args(const Args& a) {
    asm volatile("" ::"s"(a.recs), "s"(a.dvals), "s"(a.rec_stride), "s"(a.d_stride), "s"(a.d_row), "s"(a.x),
                 "s"(a.x_stride), "s"(a.x2_off), "s"(a.silu_mul), "s"(a.y), "s"(a.y_stride), "s"(a.first_mat),
                 "s"(a.probs), "s"(a.n_active), "s"(a.n_probs), "s"(a.tiles), "s"(a.units), "s"(a.rows),
                 "s"(a.cols), "s"(a.tiles_per_wg));
}

// Waits until all of this wave's vector memory loads have returned
// (s_waitcnt vmcnt(0); expcnt and lgkmcnt left at their no-wait maxima).
// A CU returns vector loads in issue order across all of its workgroups, so
// a kernel that starts with small loads (activations, tables) and then
// streams weights waits here before the stream: a weight stream issued
// earlier by another workgroup on the same CU would otherwise hold those
// small loads back behind it.
__device__ __forceinline__ void vm_wait_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Raw buffer loads. A load whose offset lies beyond the resource's size
// returns zeros without a memory access, so kernels issue every load
// unconditionally (steps past a wave's end, columns past the vector's end)
// and the compiler's load counters stay exact: vector-load waits complete in
// issue order, and a load under a branch makes every later wait count as if
// it had not been issued. Resources here are below 2 GiB, so kBufOob is out
// of range for all of them.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
constexpr uint32_t kBufWord3 = 0x00020000u;  // word 3 of a raw buffer resource (32-bit data format)
constexpr uint32_t kBufOob = 0x80000000u;
__device__ __forceinline__ BufRsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, (int)kBufWord3);
}
// Cache policy of a load: kCacheNormal, or kCacheStream (non-temporal) for
// data read exactly once (weights), so that it does not evict the small
// shared data (activations, grid) that every workgroup reads. kCacheDevice
// (sc1, device scope) reads data that another XCD's workgroup wrote during
// the same launch: each XCD has its own L2, and a plain load could return a
// line that L2 still holds from before the write.
constexpr int kCacheNormal = 0;
constexpr int kCacheStream = 2;
constexpr int kCacheDevice = 16;
template <int POL = kCacheNormal>
__device__ __forceinline__ uint4 buf_load_b128(BufRsrc r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POL);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
template <int POL = kCacheNormal>
__device__ __forceinline__ uint2 buf_load_b64(BufRsrc r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, POL);
    return make_uint2(v[0], v[1]);
}
template <int POL = kCacheNormal>
__device__ __forceinline__ uint32_t buf_load_b32(BufRsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, POL);
}
template <int POL = kCacheNormal>
__device__ __forceinline__ uint16_t buf_load_b16(BufRsrc r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, POL);
}

// Problem p of a GEMV launch with an optional device problem list (probs:
// {matrix, x row, y row, 0} per problem; n_active: its count): false when the
// count leaves p out of this call. Without a list (both null) nothing is
// read: the branch is uniform, so the first weight load waits for no vector
// round trip. With one, the count and the entry load together and one wait
// covers both (the asm needs both values before either is used; a null
// pointer is a zero-size resource, whose load returns zeros).
__device__ __forceinline__ bool read_problem(const uint4* probs, const uint32_t* n_active, uint32_t p, uint64_t& mat,
                                             uint64_t& x_row, uint64_t& y_row) {
    if (!probs && !n_active) return true;
    uint32_t n_act = buf_load_b32(make_rsrc(n_active, n_active ? 4u : 0u), 0, 0);
    uint4 d = buf_load_b128(make_rsrc(probs, probs ? (p + 1) * 16u : 0u), p * 16u, 0);
    asm volatile("" : "+v"(n_act), "+v"(d.x), "+v"(d.y), "+v"(d.z));
    if (n_active && p >= __builtin_amdgcn_readfirstlane(n_act)) return false;
    if (probs) {
        mat = __builtin_amdgcn_readfirstlane(d.x);
        x_row = __builtin_amdgcn_readfirstlane(d.y);
        y_row = __builtin_amdgcn_readfirstlane(d.z);
    }
    return true;
}

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// The IQ2_XXS grid (dequant.zig:148-213): 256 entries of 8 magnitudes.
static __constant__ uint64_t c_iq2_grid[256] = {
#include "../iq2xxs_grid.inc"
};
constexpr uint64_t kIq2Grid[256] = {
#include "../iq2xxs_grid.inc"
};

// 0xFF in every byte whose bit is set in the 4-bit sign nibble m.
__host__ __device__ constexpr uint32_t nibble_byte_mask(uint32_t m) {
    return ((m & 1u) ? 0xFFu : 0u) | ((m & 2u) ? 0xFF00u : 0u) | ((m & 4u) ? 0xFF0000u : 0u) |
           ((m & 8u) ? 0xFF000000u : 0u);
}
__host__ __device__ constexpr uint32_t parity3(uint32_t v) { return (v ^ (v >> 1) ^ (v >> 2)) & 1u; }
// Negates the bytes selected by mask (0xFF per byte). Grid magnitudes are at
// most 0x2B, so (b ^ 0xFF) + 1 never carries into the next byte.
__host__ __device__ constexpr uint32_t negate_bytes(uint32_t w, uint32_t mask) {
    return (w ^ mask) + (mask & 0x01010101u);
}

// Byte mask (0xFF per byte to negate) of columns 4..7 for hi3 = h: columns
// 4..6 take h's bits, column 7 its parity (the ksigns parity bit; column 7's
// P sign is already in the record entry).
__host__ __device__ constexpr uint32_t iq2_hi3_mask(uint32_t h) { return nibble_byte_mask(h | (parity3(h) << 3)); }

// IQ2_XXS B operands of the two records in one tile dword, from the LDS
// record entries and hi3 masks (tab: kIq2LdsWords words). The mask table
// holds 8 entries (mask, mask & 0x01010101) keyed by hi3, so the signs cost
// one xor-add, (w ^ m) + (m & 0x01010101) (negate_bytes with the second term
// read instead of computed). The mask reads touch at most 16 words:
// broadcasts without bank conflicts.
__device__ __forceinline__ long iq2_bop(uint32_t entry_off, uint32_t mask_off, const uint32_t* __restrict__ tab) {
    const char* t8 = reinterpret_cast<const char*>(tab);
    const uint2 e = *reinterpret_cast<const uint2*>(t8 + entry_off);
    const uint2 m = *reinterpret_cast<const uint2*>(t8 + kIq2TableWords * 4 + mask_off);
    return (long)(((uint64_t)((e.y ^ m.x) + m.y) << 32) | (uint64_t)e.x);
}
// Sub-block 2k: entry at bits 3..14, hi3 at bits 15..17.
__device__ __forceinline__ long iq2_bop_lo(uint32_t d, const uint32_t* __restrict__ tab) {
    return iq2_bop(d & 0x7FF8u, (d >> 12) & 0x38u, tab);
}
// Sub-block 2k + 1: entry at bits 18..29, hi3 at bits 0..2.
__device__ __forceinline__ long iq2_bop_hi(uint32_t d, const uint32_t* __restrict__ tab) {
    return iq2_bop((d >> 15) & 0x7FF8u, (d << 3) & 0x38u, tab);
}

// ls of sub-block g (from dwords 0,1) and 4+g (dwords 2,3) of this lane.
__device__ __forceinline__ uint32_t iq2_ls_a(const uint4& r) { return (r.x >> 30) | ((r.y >> 30) << 2); }
__device__ __forceinline__ uint32_t iq2_ls_b(const uint4& r) { return (r.z >> 30) | ((r.w >> 30) << 2); }

// All eight 4-bit ls values of the lane's row (nibble s = sub-block s),
// gathered from the row's four lanes (lane groups g = 0..3) by OR-ing over
// 16-lane rows with two permlane swaps: permlane16_swap(m, m) returns rows
// (0,0,2,2) and (1,1,3,3) of m, permlane32_swap(m, m) rows (0,1,0,1) and
// (2,3,2,3). No LDS traffic.
__device__ __forceinline__ uint32_t iq2_ls_all(const uint4& r, uint32_t g) {
    const uint32_t mine = (iq2_ls_a(r) << (4 * g)) | (iq2_ls_b(r) << (16 + 4 * g));
    const auto p = __builtin_amdgcn_permlane16_swap(mine, mine, false, false);
    const uint32_t pair = p[0] | p[1];
    const auto q = __builtin_amdgcn_permlane32_swap(pair, pair, false, false);
    return q[0] | q[1];
}

// Exact integer value of one MFMA output for the (hi, lo) digit rows:
// |256 D_hi + D_lo| <= 256*32*127*127 + 32*127*128 < 2^31.
__device__ __forceinline__ int digits_combine(int d_hi, int d_lo) { return d_hi * 256 + d_lo; }

// Row r (16 lanes) of the result holds v_r's lanes 0..15: four values that
// live in lanes 0..15 of four VGPRs end up one per 16-lane row.
__device__ __forceinline__ int gather_rows4(int v0, int v1, int v2, int v3) {
    auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v0, (uint32_t)v1, false, false);  // [v0 r0, v1 r0, v0 r2, v1 r2]
    auto q = __builtin_amdgcn_permlane16_swap((uint32_t)v2, (uint32_t)v3, false, false);  // [v2 r0, v3 r0, v2 r2, v3 r2]
    auto r = __builtin_amdgcn_permlane32_swap(p[0], q[0], false, false);                  // [v0 r0, v1 r0, v2 r0, v3 r0]
    return (int)r[0];
}

// The 32 KiB record table (layout above), generated at compile time from
// the grid: entry (b012 | P<<3 | idx<<4) = words (columns 0..3 of grid entry
// idx with signs b012 and P ^ parity(b012); columns 4..7 with column 7
// negated when P is set).
struct Iq2Tables {
    uint32_t w[kIq2TableWords];
};
constexpr Iq2Tables make_iq2_tables() {
    Iq2Tables t{};
    for (uint32_t e = 0; e < 4096; ++e) {
        const uint32_t b012 = e & 7u, par = (e >> 3) & 1u, idx = e >> 4;
        const uint32_t lo = (uint32_t)kIq2Grid[idx], hi = (uint32_t)(kIq2Grid[idx] >> 32);
        t.w[2 * e] = negate_bytes(lo, nibble_byte_mask(b012 | ((par ^ parity3(b012)) << 3)));
        t.w[2 * e + 1] = negate_bytes(hi, nibble_byte_mask(par << 3));
    }
    return t;
}
static __constant__ Iq2Tables c_iq2_tables = make_iq2_tables();

// LDS copy of the tables for a workgroup of WG threads, in two halves so the
// loads can be issued with the kernel's other small loads: thread t moves the
// 16-byte words t + WG * i (consecutive lanes, consecutive words: no LDS bank
// conflicts). The caller waits for the loads between the halves and
// synchronises before the first lookup.
template <int WG>
struct Iq2TableCopy {
    static constexpr int kPerThread = kIq2TableWords / 4 / WG;
    static_assert(kIq2TableWords / 4 % WG == 0, "table copy needs WG | 2048");
    uint4 v[kPerThread];
    __device__ __forceinline__ void load() {
        const BufRsrc r = make_rsrc(&c_iq2_tables, sizeof(Iq2Tables));
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) v[i] = buf_load_b128(r, (threadIdx.x + WG * i) * 16, 0);
    }
    // tab: kIq2LdsWords words (record entries, then the hi3 masks).
    __device__ __forceinline__ void store(uint32_t* tab) const {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) reinterpret_cast<uint4*>(tab)[threadIdx.x + WG * i] = v[i];
        if (threadIdx.x < kIq2MaskWords) {
            const uint32_t m = iq2_hi3_mask(threadIdx.x >> 1);
            tab[kIq2TableWords + threadIdx.x] = (threadIdx.x & 1) ? m & 0x01010101u : m;
        }
    }
};

// Wave-wide sum (all 64 lanes receive the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Quantise one 32-element block held one element per lane of a 32-lane half
// wave: returns this lane's digits and the block scale (same in all 32 lanes).
// Blocks whose max |x| is non-finite get a NaN scale (the block then poisons
// every output that reads it); blocks below 2^-100 are treated as zero.
__device__ __forceinline__ float quantize_block32(float x, int8_t* hi, int8_t* lo) {
    // NaN counts as Inf so that fmaxf (which drops NaN operands) cannot hide it.
    float a = (x != x) ? __uint_as_float(0x7F800000u) : fabsf(x);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float scale, inv;
    if (!(a <= 3.4028235e38f)) {
        scale = __uint_as_float(0x7FC00000u);
        inv = 0.0f;
    } else if (a < 0x1p-100f) {
        scale = 0.0f;
        inv = 0.0f;
    } else {
        scale = a * (1.0f / kDigitMax);
        inv = __builtin_amdgcn_rcpf(scale);
    }
    float qf = rintf(x * inv);
    qf = fminf(fmaxf(qf, -kDigitMax), kDigitMax);
    int q = (inv == 0.0f) ? 0 : (int)qf;
    int h = (q + 128) >> 8;
    *hi = (int8_t)h;
    *lo = (int8_t)(q - h * 256);
    return scale;
}

// Wave-wide max (every lane receives it) with DPP and the row permutes:
// within quads, half rows and rows, then across row pairs and halves. All
// VALU; no LDS round trip. NaN-free inputs (the caller checks).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}

// Max over each aligned group of 8 lanes (DPP: quad swaps, then the
// half-row mirror); every lane of the group receives it. All 64 lanes must be
// active.
__device__ __forceinline__ float max8_lanes(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    return v;
}

// The same maxima for non-negative inputs (+Inf and positive NaN patterns
// allowed): such floats order as their bit patterns do (a NaN above +Inf), so
// the max is an integer max of the bits, which DPP feeds directly (no
// canonicalising moves between steps).
template <int CTRL>
__device__ __forceinline__ uint32_t umax_dpp(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
    return v > o ? v : o;
}
__device__ __forceinline__ float max8_lanes_nonneg(float x) {
    uint32_t v = __float_as_uint(x);
    v = umax_dpp<0xB1>(v);
    v = umax_dpp<0x4E>(v);
    v = umax_dpp<0x141>(v);
    return __uint_as_float(v);
}
__device__ __forceinline__ float wave_max_nonneg(float x) {
    uint32_t v = __float_as_uint(x);
    v = umax_dpp<0xB1>(v);
    v = umax_dpp<0x4E>(v);
    v = umax_dpp<0x141>(v);
    v = umax_dpp<0x140>(v);
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = p[0] > p[1] ? p[0] : p[1];
    const auto q = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return __uint_as_float(q[0] > q[1] ? q[0] : q[1]);
}

// Activation quantisation for the decode kernels: one 32-column block per 8
// lanes, 4 columns per lane. A block's scale is s = max|x| / 32512 and each
// column becomes q = rint(x / s) in [-32512, 32512], split into int8 digits
// hi = (q + 128) >> 8 and lo = q - 256 hi (x ~= s (256 hi + lo)). Blocks whose
// max |x| is non-finite (NaN counts as Inf) get a NaN scale, which poisons
// every output that reads them; blocks below 2^-100 are all zero. The
// reciprocal need not be correctly rounded: q is clamped, and the error stays
// far below the half-step rounding error.
//
// The largest |x| of this lane's four columns as bits: |x| of a finite or
// infinite x orders as its bit pattern, and a NaN's pattern lies above +Inf,
// so the block's maximum is non-finite exactly when one of its x is.
__device__ __forceinline__ uint32_t quad_abs_max_bits(const float (&v)[4]) {
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t a = __float_as_uint(v[e]) & 0x7FFFFFFFu;
        m = a > m ? a : m;
    }
    return m;
}
// Scale and reciprocal of a block from its max |x| (bits); inv = 0 marks a
// block whose digits are all zero.
__device__ __forceinline__ float quad_scale(uint32_t m_bits, float& inv) {
    const float m = __uint_as_float(m_bits);
    const bool bad = m_bits >= 0x7F800000u;  // Inf or NaN
    const bool tiny = m < 0x1p-100f;
    const float sc = m * (1.0f / kDigitMax);
    const float iv = __builtin_amdgcn_rcpf(sc);
    inv = (bad || tiny) ? 0.0f : iv;
    return bad ? __uint_as_float(0x7FC00000u) : (tiny ? 0.0f : sc);
}
// The four columns' digits: with q' = q + 128 (|q'| < 2^15), hi is byte 1 of
// q' and lo is byte 0 of q' with its top bit flipped ((q' mod 256) - 128 =
// q - 256 hi), so two byte permutes gather the four q' into 16-bit pairs and
// two more pick the hi and the lo bytes.
__device__ __forceinline__ void quad_digits(const float (&v)[4], float inv, uint32_t& hi4, uint32_t& lo4) {
    int q[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) q[e] = (int)fminf(fmaxf(rintf(v[e] * inv), -kDigitMax), kDigitMax) + 128;
    const uint32_t a = __builtin_amdgcn_perm((uint32_t)q[1], (uint32_t)q[0], 0x05040100u);
    const uint32_t b = __builtin_amdgcn_perm((uint32_t)q[3], (uint32_t)q[2], 0x05040100u);
    const bool zero = inv == 0.0f;
    hi4 = zero ? 0u : __builtin_amdgcn_perm(b, a, 0x07050301u);
    lo4 = zero ? 0u : __builtin_amdgcn_perm(b, a, 0x06040200u) ^ 0x80808080u;
}
__device__ __forceinline__ float quantize_quad(const float (&v)[4], uint32_t& hi4, uint32_t& lo4) {
    float inv;
    const float scale = quad_scale(__float_as_uint(max8_lanes_nonneg(__uint_as_float(quad_abs_max_bits(v)))), inv);
    quad_digits(v, inv, hi4, lo4);
    return scale;
}

// Quantisation of 4 columns per lane with one scale for the whole wave
// (256 columns): the block fixed point of quantize_quad with the max taken
// over 64 lanes. Used where the consumer applies one activation scale per
// 256-column record unit (the grouped IQ2_XXS matmul).
__device__ __forceinline__ float quantize_quad_wave(const float (&v)[4], uint32_t& hi4, uint32_t& lo4) {
    float inv;
    const float scale = quad_scale(__float_as_uint(wave_max_nonneg(__uint_as_float(quad_abs_max_bits(v)))), inv);
    quad_digits(v, inv, hi4, lo4);
    return scale;
}

// A pass covers WG / 8 blocks: thread t quantises columns 4 (t & 7) .. +3 of
// block b0 + t / 8. x_pass_load issues the loads (xr covers the vector's
// cols floats; columns beyond read as zero), x_pass_store quantises into the
// LDS A layout (kAGroupBytes per 256 columns) and the block scales xs[];
// blocks at or beyond nblk are not stored. Every thread of the block must
// call both (the max uses DPP).
__device__ __forceinline__ void x_pass_load(BufRsrc xr, uint32_t b0, float (&v)[4]) {
    const uint32_t off = ((b0 + (threadIdx.x >> 3)) * 32 + 4 * (threadIdx.x & 7)) * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(buf_load_b32(xr, off + 4 * e, 0));
}
// silu(x) = x / (1 + exp(-x))  (math.zig:38-41).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// Wide activation quantisation by one wave: unit u (256 columns, 4 per lane)
// of vector v of src (silu(g) * g[u_off + col] when SILU) into the digit
// planes, its scale stored in the unit's eight block slots.
template <bool SILU>
__device__ __forceinline__ void quantize_unit_wave(const float* __restrict__ src, uint64_t src_stride, uint64_t u_off,
                                                   uint64_t v, uint32_t u, uint32_t cols, int8_t* __restrict__ hi,
                                                   int8_t* __restrict__ lo, float* __restrict__ sc, uint64_t q_stride,
                                                   uint64_t s_stride) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t c0 = u * 256 + lane * 4;
    const float* g = src + v * src_stride;
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t col = c0 + e;
        x[e] = 0.0f;
        if (col < cols) x[e] = SILU ? silu(g[col]) * g[u_off + col] : g[col];
    }
    uint32_t h4, l4;
    const float s = quantize_quad_wave(x, h4, l4);
    *reinterpret_cast<uint32_t*>(hi + v * q_stride + c0) = h4;
    *reinterpret_cast<uint32_t*>(lo + v * q_stride + c0) = l4;
    if (lane < 8) sc[v * s_stride + u * 8 + lane] = s;
}


// v = silu(v) * u elementwise (expertFFN's siluInplace + mul, inference.zig:1179-1180).
__device__ __forceinline__ void silu_mul4(float (&v)[4], const float (&u)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = silu(v[e]) * u[e];
}

__device__ __forceinline__ void x_pass_store(const float (&v)[4], uint32_t nblk, uint32_t b0, int8_t* aq, float* xs) {
    uint32_t h4, l4;
    const float s = quantize_quad(v, h4, l4);
    const uint32_t b = b0 + (threadIdx.x >> 3), jq = threadIdx.x & 7;
    if (b < nblk) {
        int8_t* run = aq + (b >> 3) * kAGroupBytes + (jq >> 1) * kARun + (b & 7) * 8 + 4 * (jq & 1);
        *reinterpret_cast<uint32_t*>(run) = h4;
        *reinterpret_cast<uint32_t*>(run + 4 * kARun) = l4;
        if (jq == 0) xs[b] = s;
    }
}
// Whole activation chunk: blocks [0, nblk) of the vector behind xr (times
// silu: silu(x) * u with u behind ur).
template <int WG>
__device__ __forceinline__ void quantize_to_lds(BufRsrc xr, BufRsrc ur, bool silu_mul, uint32_t nblk, int8_t* aq,
                                                float* xs) {
    for (uint32_t b0 = 0; b0 < nblk; b0 += WG / 8) {
        float v[4], u[4];
        x_pass_load(xr, b0, v);
        x_pass_load(ur, b0, u);
        if (silu_mul) silu_mul4(v, u);
        x_pass_store(v, nblk, b0, aq, xs);
    }
}

// The 8 A operands (blocks 8G..8G+7 of the LDS chunk) of a lane with
// n = m < 2: four 128-bit reads of its 64-byte run.
__device__ __forceinline__ void lds_a_group(long (&areg)[8], const int8_t* a_run, uint32_t group) {
    const uint4* p = reinterpret_cast<const uint4*>(a_run + group * kAGroupBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 q = p[i];
        areg[2 * i] = (long)(((uint64_t)q.y << 32) | q.x);
        areg[2 * i + 1] = (long)(((uint64_t)q.w << 32) | q.z);
    }
}

}  // namespace mmhip
