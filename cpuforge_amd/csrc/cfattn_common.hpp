// Shared device code for the cfattn gfx950 kernels: types, MFMA wrappers,
// bf16 rounding, workgroup-id remapping and LDS tile staging.
//
// MFMA lane layouts used throughout (checked on gfx950 for all four builtins):
//   v_mfma_f32_32x32x16_bf16: lane l holds A[l%32][8*(l/32)+0..7] and
//       B[8*(l/32)+0..7][l%32]; the 16 accumulators of lane l are
//       C[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
//   v_mfma_f32_32x32x2f32:    lane l holds A[l%32][l/32], B[l/32][l%32];
//       same accumulator layout.
// The k-index inside one MFMA may be permuted freely as long as A and B use
// the same permutation; the kernels use that to feed accumulator registers
// of one MFMA straight into the next one as operands.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cfattn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t bf16_bits;  // bf16 values live in memory as raw 16-bit patterns

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ----------------------------------------------------------------- modes
// Mode<float>: fp32 parity mode (v_mfma_f32_32x32x2f32, one element per lane
// per MFMA).  Mode<bf16_bits>: bf16 inputs, fp32 accumulation
// (v_mfma_f32_32x32x16_bf16, eight elements per lane per MFMA).
template <typename T>
struct Mode;

template <>
struct Mode<float> {
    static constexpr int EPL = 1;  // operand elements per lane per MFMA
    static constexpr int CH = 4;   // elements per 16-byte chunk
    using frag = float;
};

template <>
struct Mode<bf16_bits> {
    static constexpr int EPL = 8;
    static constexpr int CH = 8;
    using frag = bf16x8;
};

__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// A wave-uniform value moved to a scalar register.  Called through this
// device function: hipcc's host pass drops a kernel (an undefined launch stub)
// whose body names the builtin directly.
__device__ __forceinline__ int wave_uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Compile-time tag selecting one code path of a kernel (a wave role).
template <bool B>
struct RoleTag {
    static constexpr bool value = B;
};

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; i++) z[i] = 0.0f;
    return z;
}

// Round-to-nearest-even f32 -> bf16 bit pattern (finite inputs and inf; NaN
// is kept a quiet NaN).
__host__ __device__ __forceinline__ bf16_bits f32_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_bits)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (bf16_bits)(u >> 16);
}
__host__ __device__ __forceinline__ float bf16_to_f32(bf16_bits b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}

template <typename T>
__device__ __forceinline__ float to_f32(T x);
template <>
__device__ __forceinline__ float to_f32<float>(float x) {
    return x;
}
template <>
__device__ __forceinline__ float to_f32<bf16_bits>(bf16_bits x) {
    return bf16_to_f32(x);
}

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) {
    return x;
}
template <>
__device__ __forceinline__ bf16_bits from_f32<bf16_bits>(float x) {
    return f32_to_bf16(x);
}

// Eight consecutive bf16 from 16-byte-aligned memory as an MFMA operand.
__device__ __forceinline__ bf16x8 load_bf16x8(const bf16_bits* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}
// Two groups of four consecutive bf16 (each 8-byte aligned) as one operand.
__device__ __forceinline__ bf16x8 load_bf16x4x2(const bf16_bits* p0, const bf16_bits* p1) {
    uint2 a = *reinterpret_cast<const uint2*>(p0);
    uint2 b = *reinterpret_cast<const uint2*>(p1);
    uint4 v = make_uint4(a.x, a.y, b.x, b.y);
    return __builtin_bit_cast(bf16x8, v);
}
// Eight f32 accumulator values rounded to bf16 as one operand.
__device__ __forceinline__ bf16x8 pack_bf16x8(const float* v) {
    uint4 u;
    u.x = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
    u.y = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
    u.z = (uint32_t)f32_to_bf16(v[4]) | ((uint32_t)f32_to_bf16(v[5]) << 16);
    u.w = (uint32_t)f32_to_bf16(v[6]) | ((uint32_t)f32_to_bf16(v[7]) << 16);
    return __builtin_bit_cast(bf16x8, u);
}

// --------------------------------------------------------- XCD remapping
// MI355X dispatches consecutive workgroup ids round-robin over its 8 XCDs,
// each with its own L2.  Remap so that XCD x runs one contiguous range of
// logical ids; the kernels order logical ids so that a range shares K/V
// heads, which then stay resident in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int hw_id, int n, int enable) {
    if (!enable || n < 8) return hw_id;
    const int q = n / 8, r = n % 8;
    const int xcd = hw_id % 8, local = hw_id / 8;
    const int start = xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q;
    return start + local;
}

// Position of logical id `id` within its XCD's run under xcd_remap (n ids,
// remapping on, n >= 8): the workgroup that runs it is local * 8 + its XCD.
__device__ __forceinline__ int xcd_local(int id, int n) {
    const int q = n / 8, r = n % 8;
    return id < r * (q + 1) ? id % (q + 1) : (id - r * (q + 1)) % q;
}

// Work unit `it` of a workgroup of a persistent grid (8 * W workgroups) over
// n_groups groups of n_units units each, unit n_units - 1 the longest (a
// query tile, or a key tile counted from the end): the XCD of workgroup w
// (w % 8; the dispatcher deals workgroups round robin) takes a contiguous run
// of the groups (sequence and KV head, or query head), so that its L2 holds
// few of their K/V or Q/dO rows, and its W workgroups walk the run's units
// in a snake (positions l, 2W - 1 - l, 2W + l, ...), which gives every
// workgroup nearly the same work: ordered longest unit first across the run
// (unit-major), or group by group, each longest first (group-major: fewer
// groups in flight at once, for the L2; persistent_group_major picks it where
// it balances as well).  (A grid of one workgroup per unit leaves CUs idle
// while units remain: units of very different lengths stall the in-order
// dispatch.)  False past the run.
__device__ __forceinline__ bool persistent_item(int it, int n_groups, int n_units, int W, int group_major, int& unit,
                                                int& grp) {
    const int xq = blockIdx.x % 8, xl = blockIdx.x / 8;
    const int q = n_groups / 8, r = n_groups % 8;
    const int g0 = xq < r ? xq * (q + 1) : r * (q + 1) + (xq - r) * q;
    const int gn = q + (xq < r ? 1 : 0);
    const int pos = (it >> 1) * 2 * W + ((it & 1) ? 2 * W - 1 - xl : xl);
    if (gn == 0 || pos >= gn * n_units) return false;
    if (group_major) {
        unit = n_units - 1 - pos % n_units;
        grp = g0 + pos / n_units;
    } else {
        unit = n_units - 1 - pos / gn;
        grp = g0 + pos % gn;
    }
    return true;
}

// ------------------------------------------------------------ LDS staging
template <typename T>
union Chunk {
    uint4 u;
    T e[16 / sizeof(T)];
};

// Copy rows [0, ROWS) x columns [0, DP) of a strided global tile into LDS,
// row-major with leading dimension LD (elements).  Rows at or past `nrows`
// and columns at or past `hd` are written as zero, so padded rows and
// head-dim padding contribute nothing to any contraction.
template <typename T, int ROWS, int DP, int LD>
__device__ __forceinline__ void stage_rows(T* __restrict__ s, const T* __restrict__ g, long row_stride, int nrows,
                                           int hd, bool vec_ok, int nthreads) {
    constexpr int CH = Mode<T>::CH;
    constexpr int CPR = DP / CH;  // 16-byte chunks per row
    constexpr int TOTAL = ROWS * CPR;
    for (int c = threadIdx.x; c < TOTAL; c += nthreads) {
        const int row = c / CPR;
        const int col = (c % CPR) * CH;
        Chunk<T> v;
        if (row < nrows && vec_ok && col + CH <= hd) {
            v.u = *reinterpret_cast<const uint4*>(g + (long)row * row_stride + col);
        } else {
#pragma unroll
            for (int i = 0; i < CH; i++)
                v.e[i] = (row < nrows && col + i < hd) ? g[(long)row * row_stride + col + i] : T(0);
        }
        *reinterpret_cast<uint4*>(s + row * LD + col) = v.u;
    }
}

// The same tile transposed: LDS holds element (row, d) at s[d * LD + row].
// Each thread moves four rows x one 16-byte column chunk and writes the four
// rows of each d with one store.
template <typename T, int ROWS, int DP, int LD>
__device__ __forceinline__ void stage_rows_t(T* __restrict__ s, const T* __restrict__ g, long row_stride, int nrows,
                                             int hd, bool vec_ok, int nthreads) {
    constexpr int CH = Mode<T>::CH;
    constexpr int RG = ROWS / 4;  // groups of four rows
    constexpr int TOTAL = RG * (DP / CH);
    static_assert(ROWS % 4 == 0, "row tile must be a multiple of 4");
    for (int c = threadIdx.x; c < TOTAL; c += nthreads) {
        const int r0 = (c % RG) * 4;
        const int col = (c / RG) * CH;
        Chunk<T> v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int row = r0 + j;
            if (row < nrows && vec_ok && col + CH <= hd) {
                v[j].u = *reinterpret_cast<const uint4*>(g + (long)row * row_stride + col);
            } else {
#pragma unroll
                for (int i = 0; i < CH; i++)
                    v[j].e[i] = (row < nrows && col + i < hd) ? g[(long)row * row_stride + col + i] : T(0);
            }
        }
#pragma unroll
        for (int i = 0; i < CH; i++) {
            if constexpr (sizeof(T) == 2) {
                uint2 w;
                w.x = (uint32_t)v[0].e[i] | ((uint32_t)v[1].e[i] << 16);
                w.y = (uint32_t)v[2].e[i] | ((uint32_t)v[3].e[i] << 16);
                *reinterpret_cast<uint2*>(s + (col + i) * LD + r0) = w;
            } else {
                float4 w = make_float4(v[0].e[i], v[1].e[i], v[2].e[i], v[3].e[i]);
                *reinterpret_cast<float4*>(s + (col + i) * LD + r0) = w;
            }
        }
    }
}

// Load one lane's operand row: elements [d0, d0 + N) of a global row into N
// registers (zero past hd or for an invalid row).
template <typename T, int N>
__device__ __forceinline__ void load_row_frag(T (&dst)[N], const T* __restrict__ row, int d0, int hd, bool valid,
                                              bool vec_ok) {
    constexpr int CH = Mode<T>::CH;
    static_assert(N % CH == 0, "fragment must be whole chunks");
#pragma unroll
    for (int c = 0; c < N / CH; c++) {
        const int d = d0 + c * CH;
        Chunk<T> v;
        if (valid && vec_ok && d + CH <= hd) {
            v.u = *reinterpret_cast<const uint4*>(row + d);
        } else {
#pragma unroll
            for (int i = 0; i < CH; i++) v.e[i] = (valid && d + i < hd) ? row[d + i] : T(0);
        }
#pragma unroll
        for (int i = 0; i < CH; i++) dst[c * CH + i] = v.e[i];
    }
}

// ------------------------------------------------ swizzled bf16 LDS tiles
// Fast-path tiles hold rows of DP bf16 (DP = 64 or 128) without padding; the
// 16-byte chunk c of row r is stored at chunk position c ^ swz<DP>(r).  gfx950
// LDS serves 256 bytes per clock over 64 four-byte banks, so the patterns
// below are chosen to be conflict-free for 16 lanes at a time:
//   - ds_read_b128 of one chunk column by 16 consecutive rows (MFMA operand
//     rows) lands on 16 different 16-byte bank groups;
//   - ds_read_b64_tr_b16 by lanes 0-31 (rows r0..r0+3, r0 % 4 == 0, chunks
//     c0..c0+3, c0 % 4 == 0) lands on 16 different bank groups;
//   - ds_write_b128 of whole rows is a permutation within each bank row.
// DP = 128 (one row per bank row): swz = 4*(r%4) + (r/4)%4, period 16.
// DP = 64 (two rows per bank row): swz = 4*((r/2)%2) + (r/4)%4, values 0..7,
// distinct over the eight rows of each parity in 16 consecutive rows.
template <int DP>
__device__ __forceinline__ int swz(int r) {
    if constexpr (DP == 128)
        return ((r & 3) << 2) | ((r >> 2) & 3);
    else
        return (((r >> 1) & 1) << 2) | ((r >> 2) & 3);
}
template <int DP>
__device__ __forceinline__ int swz_off(int r, int c) {
    return r * DP + ((c ^ swz<DP>(r)) << 3);
}

// ------------------------------------------------- direct-to-LDS loads
// global_load_lds_dwordx4 written as inline assembly: 64 lanes x 16 bytes
// from per-lane global addresses to 1 KiB of consecutive LDS starting at
// `lds` (wave-uniform; the instruction takes it in m0, which the compiler
// loads for the asm operand).  Unlike the builtin, the compiler does not
// see the LDS write, so it inserts no wait for it: the caller waits with
// s_waitcnt vmcnt (these loads count there, in issue order) and then
// barriers.  Used where the compiler's own tracking of several in-flight
// buffers falls back to waiting for every load.
//
// The m0 write the compiler emits for the operand needs one wait state
// before an LDS-DMA instruction reads it, which the compiler's hazard
// checks do not see through the asm: hence the s_nop 0 in each.
//
// s_waitcnt immediate (gfx9 encoding) for vmcnt(0) alone, for a wait the
// compiler's own wait-count tracking sees (__builtin_amdgcn_s_waitcnt).
constexpr int kWaitVmcnt0 = 0x0F70;  // vmcnt 0, expcnt 7, lgkmcnt 15: no wait on the others
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
__device__ __forceinline__ void lds_load16_asm(const void* g, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}
// The same with the non-temporal cache policy, for data read exactly once.
__device__ __forceinline__ void lds_load16_nt_asm(const void* g, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(m0) : "memory");
}
// The same loads addressed as a scalar base plus a 32-bit per-lane byte
// offset (the saddr form: no 64-bit address arithmetic per lane).
__device__ __forceinline__ void lds_load16_sv(const void* sbase, uint32_t voff, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void lds_load4_sv(const void* sbase, uint32_t voff, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(m0) : "memory");
}
// The same with the LDS destination given as a byte address (M0).
__device__ __forceinline__ void lds_load16_so(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ __forceinline__ void lds_load4_so(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// A raw buffer resource (gfx9 layout: 48-bit base, stride 0, num_records,
// 32-bit untyped data format): loads at byte offsets at or past num_records
// return zeros and access no memory.
typedef int32_t BufRsrc __attribute__((ext_vector_type(4)));
__device__ __forceinline__ BufRsrc buf_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    BufRsrc r;
    r[0] = (int32_t)(uint32_t)a;
    r[1] = (int32_t)(uint32_t)(a >> 32);
    r[2] = (int32_t)bytes;
    r[3] = 0x00020000;
    return r;
}
// 64 lanes x 16 bytes from a buffer (lane byte offset voff) to 1 KiB of LDS
// at byte address lds (M0), and the same for 4 bytes per lane.
__device__ __forceinline__ void lds_buf_load16(const BufRsrc& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
__device__ __forceinline__ void lds_buf_load4(const BufRsrc& r, uint32_t voff, uint32_t lds) {
    asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)) : "memory");
}
// 64 lanes x 4 bytes to 256 consecutive bytes of LDS (one float per lane).
__device__ __forceinline__ void lds_load4_asm(const void* g, const void* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
    asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(m0) : "memory");
}

// ------------------------------------------------- blocked bf16 LDS tiles
// A tile of ROWS rows of DP bf16 (DP = 64 or 128) filled by direct-to-LDS
// loads: one global_load_lds of 64 lanes x 16 bytes writes 1 KiB at
// consecutive addresses.  Load block b (b < NB = ROWS*DP/512) holds the rows
// b, b + NB, b + 2*NB, ... and blocks start 1040 bytes apart, so row r starts
// at element row(r) = (r % NB) * 520 + (r / NB) * DP.  Reads are then
// conflict-free on the 64 four-byte banks, and each lane's address is a base
// register plus a compile-time offset:
//   - ds_read_b128 by 16 lanes of 16 consecutive rows (one 16-byte chunk
//     each): 1040 = 16 (mod 256), so rows with distinct r % 16 start on
//     distinct 16-byte bank groups (DP = 64: r / NB adds 128 to the second
//     eight);
//   - ds_read_b64_tr_b16 by 32 lanes of four rows 4 apart, 64 bytes each:
//     the four row starts are 64 bytes apart (mod 256).
// The MFMA row i of a 32-row block is tile row qperm(i) of that block, which
// makes the four rows of every transposed read (MFMA rows 4h..4h+3 of the
// accumulator layout) 4 apart.
template <int DP, int ROWS>
struct BlkTile {
    static constexpr int NB = ROWS * DP / 512;  // load blocks
    static constexpr int STRIDE = 520;          // elements between blocks
    static constexpr int SIZE = NB * STRIDE;
    static constexpr int ROW16 = 16 / NB * DP;  // row(r + 16) - row(r)
    static_assert(NB == 8 || NB == 16, "16 rows must cover every block once or twice");
    __host__ __device__ static int row(int r) { return (r % NB) * STRIDE + (r / NB) * DP; }
};
// qperm(i) = 4*(i%4) + (i/4)%4 + 16*(i/16) on 0..31; qperm(qperm(i)) = i.
__host__ __device__ __forceinline__ constexpr int qperm(int i) { return ((i & 3) << 2) | ((i >> 2) & 3) | (i & 16); }

// max / sum of x over lanes l and l ^ 32 with one v_permlane32_swap (no LDS
// traffic, unlike a shuffle): swapping the upper half of one copy of x with
// the lower half of another leaves x[l] in one register and x[l ^ 32] in the
// other.  Written as inline asm: this compiler folds max(r0, r1) of the
// builtin's two results to r0.  The s_nop covers the VALU-write to permlane
// read hazard for the copies.
__device__ __forceinline__ void swap_halves(float x, float& a, float& b) {
    float u = x, w = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(u), "+v"(w));
    a = u;
    b = w;
}
__device__ __forceinline__ float max_halves(float x) {
    float a, b;
    swap_halves(x, a, b);
    return fmaxf(a, b);
}
__device__ __forceinline__ float sum_halves(float x) {
    float a, b;
    swap_halves(x, a, b);
    return a + b;
}

// Hardware round-to-nearest-even pack of eight f32 values into an MFMA
// operand (v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16x8 cvt_bf16x8(const float* v) {
    bf16x8 r;
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = (__bf16)v[i];
    return r;
}

// Transposed LDS read (ds_read_b64_tr_b16).  Within each group of 16 lanes,
// output lane i, element k (k = 0..3) is element i % 4 of the 8-byte row whose
// address lane 4*k + i/4 supplies.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s16x4 ds_read_tr16(const bf16_bits* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}
__device__ __forceinline__ bf16x8 join_bf16x4(s16x4 a, s16x4 b) {
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    s16x8 v = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return __builtin_bit_cast(bf16x8, v);
}

// Leading dimensions with padding chosen so that the MFMA operand reads
// (16-byte row reads for row-major tiles, 8/16-byte reads of four
// consecutive rows for transposed tiles) spread over all LDS banks.
template <typename T, int DP>
struct RowLD {
    static constexpr int value = DP + 16 / (int)sizeof(T);
};
template <typename T, int ROWS>
struct TLD {
    static constexpr int value = ROWS + (sizeof(T) == 2 ? 4 : 4);
};

}  // namespace cfattn
