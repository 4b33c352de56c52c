// Cross-lane exchanges without LDS.
//
// v_permlane32_swap / v_permlane16_swap exchange halves of two registers in place:
//   swap32(a, b): lanes 32-63 of a <-> lanes 0-31 of b
//   swap16(a, b): odd 16-lane rows of a <-> even 16-lane rows of b
// They are issued through inline assembly with both operands read-write: the compiler
// builtins for these instructions return two values, and the ROCm 7.2 compiler has been
// seen to hand back the first value for both in some contexts.  s_nop 1 before and after
// covers the VALU-write / permlane-read hazards the compiler does not see inside asm.
#pragma once

namespace tgm {

__device__ __forceinline__ void swap32(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(unsigned& a, unsigned& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(float& a, float& b) {
  unsigned x = __builtin_bit_cast(unsigned, a), y = __builtin_bit_cast(unsigned, b);
  swap32(x, y);
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}
__device__ __forceinline__ void swap16(float& a, float& b) {
  unsigned x = __builtin_bit_cast(unsigned, a), y = __builtin_bit_cast(unsigned, b);
  swap16(x, y);
  a = __builtin_bit_cast(float, x);
  b = __builtin_bit_cast(float, y);
}

// DPP exchanges inside 16-lane rows: lane l receives lane l ^ m.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float xor1(float v) { return dpp<0xB1>(v); }              // quad_perm [1,0,3,2]
__device__ __forceinline__ float xor2(float v) { return dpp<0x4E>(v); }              // quad_perm [2,3,0,1]
__device__ __forceinline__ float xor4(float v) { return dpp<0x1B>(dpp<0x141>(v)); }  // half-row mirror, quad xor 3
__device__ __forceinline__ float xor8(float v) { return dpp<0x128>(v); }             // row rotate right by 8

}  // namespace tgm
