// The gemv_rc code object: the u8 GEMV tilings of w8a16_gemv.hip with the
// reference's cast point, bf16((u - 128) * s) per weight before the product
// (crates/rxla-nn/src/layers.rs:277-296). Kernel names rxw8_gemv_rc_*.
#define RXW8_GEMV_RC 1
#include "w8a16_gemv.hip"
