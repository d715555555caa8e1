// Shared device helpers of the gfx950 expert path: number-format codecs (bit-exact with
// the build's CPU oracle), vector types and launch-check macros.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

#include "../../include/afd.h"

namespace afd {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr float kE4m3Max = 448.0f;
constexpr float kFp8Eps = 1e-10f;
constexpr int kMxBlock = 32;
constexpr int kFp8Block = 128;

// ---------------------------------------------------------------- bf16
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round to nearest even; NaN stays a quiet NaN (the rounding of torch's .to(bfloat16)).
// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even and quiets NaNs: bit for bit the
// rounding of torch's .to(bfloat16) (checked on 2^28 fp32 patterns incl. ties and denormals).
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f_t __attribute__((ext_vector_type(2)));
// (bf16(lo) | bf16(hi) << 16) with one conversion instruction
__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
  v2bf b = __builtin_convertvector((v2f_t{lo, hi}), v2bf);
  return __builtin_bit_cast(uint32_t, b);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return static_cast<uint16_t>(pk_bf16(f, 0.0f));
}

// ---------------------------------------------------------------- e4m3fn (OCP FP8)
// |v| <= 448 (callers clamp). Normals keep 3 significand bits, ties to even; below 2^-6
// the code is rint(|v| * 2^9) subnormal steps.
__device__ __forceinline__ uint32_t f32_to_e4m3(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 31) << 7;
  uint32_t mag = u & 0x7fffffffu;
  int e = static_cast<int>(mag >> 23) - 127;
  uint32_t code;
  if (e >= -6) {
    uint32_t man = mag & 0x7fffffu;
    uint32_t keep = man >> 20, rem = man & 0xfffffu;
    uint32_t up = (rem > 0x80000u) | ((rem == 0x80000u) & (keep & 1u));
    uint32_t m = keep + up;
    code = (static_cast<uint32_t>(e + 7 + static_cast<int>(m >> 3)) << 3) | (m & 7u);
  } else {
    code = static_cast<uint32_t>(__builtin_rintf(__uint_as_float(mag) * 512.0f));
  }
  return code | sign;
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  uint32_t s = (c >> 7) & 1u, e = (c >> 3) & 15u, m = c & 7u;
  float mag = e == 0 ? static_cast<float>(m) * (1.0f / 512.0f)
                     : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -mag : mag;
}

// ---------------------------------------------------------------- E2M1 (fp4)
// Input already divided by the block scale. Ties (.25 .75 1.25 1.75 2.5 3.5 5) go to
// the even code; saturates at 6.
__device__ __forceinline__ uint32_t f32_to_e2m1(float v) {
  float a = fabsf(v);
  uint32_t code = (a > 0.25f) + (a >= 0.75f) + (a > 1.25f) + (a >= 1.75f) + (a > 2.5f) +
                  (a >= 3.5f) + (a > 5.0f);
  return code | ((__float_as_uint(v) >> 31) << 3);
}

// ---------------------------------------------------------------- MX (UE8M0 per 32) scale
// Shared exponent floor(log2(amax)) - emax, clamped to [-127, 127]; amax == 0 -> code 0.
__device__ __forceinline__ uint32_t mx_scale_code(float amax, int emax) {
  if (amax == 0.0f) return 0u;
  int exp32 = static_cast<int>((__float_as_uint(amax) >> 23) & 0xffu);
  int e = exp32 > 0 ? exp32 - 127 : -127;
  int code = e - emax + 127;
  code = code < 0 ? 0 : (code > 254 ? 254 : code);
  return static_cast<uint32_t>(code);
}

// 2^(127 - code) as an exact fp32 power of two (code <= 253).
__device__ __forceinline__ float mx_inv_scale(uint32_t code) {
  return __uint_as_float((254u - code) << 23);
}

__device__ __forceinline__ float clamp_e4m3(float v) {
  return fminf(fmaxf(v, -kE4m3Max), kE4m3Max);
}

// Two clamped fp32 -> e4m3fn bytes in the low 16 bits, by v_cvt_pk_fp8_f32 (round to nearest
// even; bit-identical to f32_to_e4m3 on every fp32 input in [-448, 448]).
__device__ __forceinline__ uint32_t pk_e4m3(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(clamp_e4m3(lo), clamp_e4m3(hi), 0, false)) &
         0xffffu;
}

// Exchange between the lane halves of a wavefront: lane l < 32 receives hi_sends of lane
// l + 32, lane l >= 32 receives lo_sends of lane l - 32 (lk = l / 32). One
// v_permlane32_swap (VALU) instead of a ds_bpermute through the LDS crossbar.
// The value x, opaque to the optimizer: what is computed from the result inside a loop stays
// there instead of being hoisted out and kept live in a register across the whole loop.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ uint32_t swap_halves(uint32_t lo_sends, uint32_t hi_sends, int lk) {
  const auto r = __builtin_amdgcn_permlane32_swap(hi_sends, lo_sends, false, false);
  return lk ? r[0] : r[1];
}
__device__ __forceinline__ float xor32(float v, int lk) {
  return __uint_as_float(swap_halves(__float_as_uint(v), __float_as_uint(v), lk));
}

// x / s rounded to nearest even, bit for bit the IEEE quotient, given y = 1 / s (itself the
// IEEE quotient, computed once per divisor): q0 = x y, then one correction with the exact
// residual x - q0 s (Markstein's division step). The residual is formed negated,
// t = q0 s - x, and the correction adds -t y: the negations are operand modifiers, and a zero x
// keeps its sign through both fused steps (-0 / s stays -0; for any other x a zero residual
// leaves q0 unchanged whatever its sign). Checked on the GPU for all 2^46 pairs of fp32
// significands in [1, 2); scaling x and s by powers of two scales every step exactly, which
// carries it to every normal operand, and the FP8 quantizers' operands stay normal wherever the
// e4m3 code is not zero (s >= 1e-10 / 448). Three VALU operations per quotient instead of the
// ten of a full division.
__device__ __forceinline__ float div_by(float x, float s, float y) {
  const float q0 = x * y;
  const float t = __builtin_fmaf(q0, s, -x);
  return __builtin_fmaf(-t, y, q0);
}

// Four clamped fp32 -> four e4m3fn bytes (element i in byte i).
__device__ __forceinline__ uint32_t pk4_e4m3(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(clamp_e4m3(a), clamp_e4m3(b), 0, false);
  return static_cast<uint32_t>(
      __builtin_amdgcn_cvt_pk_fp8_f32(clamp_e4m3(c), clamp_e4m3(d), lo, true));
}
// pk4_e4m3 for values known to lie below 464 in magnitude, without the clamp: round to
// nearest even already takes (448, 464) to 448. The FP8 1x128 quotients h / s with
// s = RN(amax / 448) stay below 448 (1 + 2^-23): the FP8 gate_up epilogue converts them so (the
// activation quantizer keeps the clamp, which measured faster there).
__device__ __forceinline__ uint32_t pk4_e4m3_near(float a, float b, float c, float d) {
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// f(std::integral_constant<int, 0>{}) ... f(std::integral_constant<int, N - 1>{}): an
// unrolled loop whose index is a constant expression in the body
template <int N, int I = 0, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}

// ---------------------------------------------------------------- gate_up activations
// h from the gate and up values of one intermediate column (afd_activation). tanh(x) is
// 1 - 2 / (1 + e^{2x}): one exponential and one reciprocal, and exactly +-1 once e^{2x}
// overflows or vanishes.
__device__ __forceinline__ float act_swiglu(float g, float u) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}
__device__ __forceinline__ float tanh_exp(float x) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + __expf(2.0f * x));
}
// SwiGLU with a limit: silu(min(g, L)) * clamp(u, -L, L)
__device__ __forceinline__ float act_swiglu_limit(float g, float u, float l) {
  return act_swiglu(fminf(g, l), fminf(fmaxf(u, -l), l));
}
// SiTU: L tanh(u / L) * A tanh(g / A) * sigmoid(g)
__device__ __forceinline__ float act_situ(float g, float u, float a, float inv_a, float l,
                                          float inv_l) {
  return (l * tanh_exp(u * inv_l)) * (a * tanh_exp(g * inv_a)) *
         __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}
// the activation parameters a gate_up GEMM takes from afd_moe_cfg
struct ActParams {
  int act;  // enum afd_activation
  float a, inv_a, l, inv_l;
};
inline ActParams act_params(const afd_moe_cfg& cfg) {
  ActParams p;
  p.act = cfg.activation;
  p.a = cfg.act_alpha;
  p.l = cfg.act_limit;
  p.inv_a = cfg.activation == AFD_ACT_SITU ? 1.0f / cfg.act_alpha : 0.0f;
  p.inv_l = cfg.activation == AFD_ACT_SITU ? 1.0f / cfg.act_limit : 0.0f;
  return p;
}

// Division by a launch constant d >= 1 without the division sequence:
// n / d == __umulhi(n, ceil(2^32 / d)) for every n with n * d < 2^32 (the product overshoots
// n / d by n * (ceil(2^32/d) * d - 2^32) / 2^32 / d < n / 2^32 < 1/d, which never reaches
// the next integer). 2^32 itself does not fit 32 bits, so d == 1 is encoded as 0.
inline uint32_t div_magic(uint32_t d) {
  return d <= 1 ? 0u : static_cast<uint32_t>((0x100000000ull + d - 1) / d);
}
__device__ __forceinline__ uint32_t div_by_magic(uint32_t n, uint32_t magic) {
  return magic ? __umulhi(n, magic) : n;
}

// ---------------------------------------------------------------- persistent GEMM tile walk
// Output tiles of a grouped GEMM: row tiles [0, rows) (read from device memory) x column
// tiles [0, ntn). The dispatcher deals workgroups to the 8 XCDs round robin (workgroup b runs
// on XCD b % 8), and each XCD has its own L2. With a grid that is a multiple of 8 and at
// least kWalkSplitRows row tiles, XCD x takes the contiguous row tiles
// [rows x / 8, rows (x + 1) / 8), else every workgroup walks all of them. The tiles of a
// walk are numbered densely (`at_dense`) in blocks of BR row tiles x 32 / BR column tiles (row
// tiles fastest inside a block; row blocks outer, column blocks inner; the last row block and
// the last column block may be partial), so the ~32 workgroups of an XCD run about one block
// at a time and share each activation slice 32 / BR ways and each weight slice BR ways in
// their L2.
//
// The dense positions are handed out in one of two ways: statically (workgroup k of a walk
// takes positions first, first + stride, ...) or dynamically, from one counter per walk (per
// XCD when the rows are split), one lane of a workgroup taking the next position with an
// atomic increment (`claim_ticket`) and `resolve` mapping positions past the last tile to
// `tiles`. The tiles then stay on the XCD whose L2 shares their operands, while a workgroup
// that starts late (its CU held by another kernel, e.g. a parked stream wait) takes fewer
// tiles instead of adding a whole round at the end. Everything but the claim itself is host
// code too, so the walk's coverage is checked on the CPU (tests/walk_model.cpp).
constexpr int kWalkSplitRows = 32;
// the dynamic walk's 8 counters (one per XCD) are this many words apart
constexpr int kWalkCounterStride = 64;

template <int BR>
struct TileWalk {
  static_assert(BR == 1 || BR == 2 || BR == 4 || BR == 8 || BR == 16 || BR == 32, "BR divides 32");
  static constexpr int kBC = 32 / BR;
  int mt0, rows_here, ntn, first, stride;
  int tiles;  // rows_here * ntn: the dense positions of at_dense
  uint32_t* ctr;
  // block / grid: this workgroup's index and the grid size; counters: for the dynamic walk, 8
  // zeroed words kWalkCounterStride apart (one per XCD)
  __host__ __device__ __forceinline__ TileWalk(int rows, int ntn_, int block, int grid,
                                               uint32_t* counters = nullptr) {
    ntn = ntn_;
    mt0 = 0;
    rows_here = rows;
    first = block;
    stride = grid;
    ctr = counters;
    if ((grid & 7) == 0 && rows >= kWalkSplitRows) {
      const int xcd = block & 7;
      mt0 = (rows * xcd) >> 3;
      rows_here = ((rows * (xcd + 1)) >> 3) - mt0;
      first = block >> 3;
      stride = grid >> 3;
      if (counters != nullptr) ctr = counters + xcd * kWalkCounterStride;
    }
    tiles = rows_here * ntn;
  }
  // the next dense position of this walk's counter, possibly past the last tile
  // (global_atomic_inc with the largest limit is a plain increment); one lane calls it
  __device__ __forceinline__ uint32_t claim_ticket() const {
    return __builtin_amdgcn_atomic_inc32(ctr, 0xffffffffu, __ATOMIC_RELAXED, "agent");
  }
  // a claimed dense position, or `tiles` if it is past the last tile
  __host__ __device__ __forceinline__ int resolve(uint32_t i) const {
    return i < static_cast<uint32_t>(tiles) ? static_cast<int>(i) : tiles;
  }
  // The tile at dense position i < tiles. Row blocks of BR row tiles (the last may have
  // fewer, vr), in each, column blocks of kBC column tiles (the last may have fewer); inside
  // a block, row tiles fastest.
  __host__ __device__ __forceinline__ void at_dense(int i, int& mt, int& nt) const {
    const int full = rows_here / BR;  // full row blocks
    int rb, vr = BR, j = i;
    if (i < full * BR * ntn) {
      rb = i / (BR * ntn);
      j = i - rb * BR * ntn;
    } else {
      rb = full;
      vr = rows_here - full * BR;
      j = i - full * BR * ntn;
    }
    const int cb = j / (vr * kBC), jj = j - cb * vr * kBC;
    mt = mt0 + rb * BR + jj % vr;
    nt = cb * kBC + jj / vr;
  }
};

// ---------------------------------------------------------------- MX GEMM operand tile images
// The MX grouped GEMMs copy their operands HBM -> LDS as contiguous "tile images": the exact
// LDS bytes of one K stage (128 K values) of one row tile, followed by the UE8M0 scales of
// those rows (4 bytes = 4 blocks of 32 per row).
//   A image (activations, 128 rows of e4m3): 128 x 128 B data, then 128 x 4 B scales.
//   B image (weights, 256 rows of e2m1):     256 x  64 B data, then 256 x 4 B scales.
// Rows are XOR-swizzled by 16-byte chunk. An MFMA operand read (ds_read_b128, one chunk of
// 32 consecutive rows per half wavefront) is served 16 lanes = 256 bytes at a time by the
// 64 banks of gfx950's LDS; the swizzle puts those 16 lanes on 16 distinct 16-byte bank
// groups (and any 8 consecutive lanes on 8 distinct groups of a 128-byte line).
constexpr int kImgData = 16384;
constexpr int kImgARows = 128, kImgBRows = 256;
constexpr int kImgA = kImgData + kImgARows * 4;  // 16896
constexpr int kImgB = kImgData + kImgBRows * 4;  // 17408
constexpr int kImgK = 128;                        // K values per image
// The W4A16 GEMMs' bf16 A block of one K stage (128 rows x 128 bf16, rows XOR-swizzled by
// 16-byte chunk; afd_gemm_a16.hip): 32 KiB, no scales.
constexpr int kImgA16 = kImgARows * kImgK * 2;
// FP8 images (FP8 128x128-block weights, and the W8A8 down GEMM's e4m3 A operand): 64 K values
// of e4m3 per row, laid out as a B image's data (img_b_off), no scales: 256 weight rows = 16
// KiB, 128 activation rows = 8 KiB. The fp32 block scales stay in tables of their own.
constexpr int kF8K = 64;
constexpr int kImgF8B = kImgBRows * kF8K;  // 16384
constexpr int kImgF8A = kImgARows * kF8K;  // 8192
// The MX GEMM copies an A image's 512 B of scales as a 1 KiB piece, reading the 512 B that
// follow; buffers of A images keep that much readable memory after their last image.
constexpr int kImgReadSlack = 512;

// The 4 UE8M0 scale bytes of a row (K blocks 0..3 of the stage) are stored in the order
// block 0, 2, 1, 3: lane half h of an MFMA operand reads the 16-bit half at byte 2h and finds
// its k-step-ks block (2 ks + h) in byte ks, which the MFMA's op_sel picks directly.
__host__ __device__ __forceinline__ int scale_byte(int j) { return ((j & 1) << 1) | (j >> 1); }

// byte offset of logical 16-byte chunk c (0..7) of row r in an A image
__host__ __device__ __forceinline__ int img_a_off(int r, int c) {
  return r * 128 + ((c ^ ((r ^ (r >> 3)) & 7)) << 4);
}
// byte offset of logical 16-byte chunk c (0..3) of row n in a B image
__host__ __device__ __forceinline__ int img_b_off(int n, int c) {
  return n * 64 + ((c ^ (((n >> 1) ^ (n >> 2)) & 3)) << 4);
}
// FP8 weights [mats][rows][cols] as images [mats][rows / 256][cols / 64]: byte offset of the
// image that holds physical row `row`, columns [col - col % 64, + 64)
__host__ __device__ __forceinline__ int64_t fp8_image_offset(int64_t mat, int64_t row, int64_t col,
                                                             int rows, int cols) {
  return ((mat * (rows / kImgBRows) + row / kImgBRows) * (cols / kF8K) + col / kF8K) *
         int64_t(kImgF8B);
}

// ---------------------------------------------------------------- direct global -> LDS copies
// gfx950 global_load_lds: lane i of the wavefront writes its 16 (or 4) bytes to LDS at
// M0 + 16*i (4*i); the global address is the uniform base plus the lane's 32-bit offset.
// Issued through inline assembly so the compiler does not drain every outstanding copy
// before each LDS read; callers wait with wait_vmcnt<N>() (vector-memory operations
// complete in issue order for loads) and a barrier before reading what they copied.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// A pointer the caller knows is wavefront-uniform, moved into scalar registers.
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
  return reinterpret_cast<const void*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ void lds_dma16(uint32_t m0, const void* base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(m0), "v"(voff),
               "s"(uniform_ptr(base))
               : "memory");
}

__device__ __forceinline__ void lds_dma4(uint32_t m0, const void* base, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2" ::"s"(m0), "v"(voff),
               "s"(uniform_ptr(base))
               : "memory");
}

// Global stores through inline assembly: the compiler neither moves, merges nor splits them,
// so a caller that counts its vector-memory instructions for s_waitcnt knows their number.
// A store of more than 8 bytes reads its data registers one cycle late, and the compiler
// does not see that hazard in inline assembly, so the s_nop keeps the next instruction from
// overwriting them first.
__device__ __forceinline__ void store16(void* p, v4i v) {
  asm volatile("global_store_dwordx4 %0, %1, off\n\ts_nop 0" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ void store8(void* p, uint32_t v) {
  asm volatile("global_store_byte %0, %1, off" ::"v"(p), "v"(v) : "memory");
}

// s_waitcnt vmcnt(N) leaving the other counters alone.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Every LDS read of this wavefront complete (lgkmcnt 0), copies left in flight.
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xc07f); }

// wait_vmcnt<N> plus every LDS read of this wavefront complete (lgkmcnt 0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lds() {
  static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit counter");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

}  // namespace afd

// Host-side helpers shared by the translation units.
namespace afd {
int set_hip_error(hipError_t e);  // records e for afd_last_hip_error(); returns AFD_ERR_HIP
}

#define AFD_CHECK_LAUNCH()                                 \
  do {                                                     \
    hipError_t _e = hipGetLastError();                     \
    if (_e != hipSuccess) return afd::set_hip_error(_e);   \
  } while (0)

#define AFD_CHECK_HIP(expr)                                \
  do {                                                     \
    hipError_t _e = (expr);                                \
    if (_e != hipSuccess) return afd::set_hip_error(_e);   \
  } while (0)
