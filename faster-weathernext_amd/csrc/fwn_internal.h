// Internal helpers shared by the host pipeline and the launchers (not part of the C ABI).
#pragma once

#include <stdint.h>

#include "fwn_attn.h"

namespace fwn {

// Thread-local error message of the C ABI.
int fail(int code, const char* fmt, ...);
void clear_error();

// Column (key) offset within a 128-wide tile of register element `el` = 16 * sb + reg held by
// lane group g (lane >> 5) in the kernels' accumulator layout. The 32x32 MFMA accumulator of
// lane l, register r holds output row 8*(r/4) + 4*(l/32) + r%4; operand rows are loaded
// permuted so that this row is key 16*(r/8) + 8*(l/32) + r%8 of the 32-key sub-block sb. Each
// lane group then holds 8 consecutive keys per 16-key chunk, which is the operand layout of the
// next MFMA (P or dS as the B operand), so probabilities never leave registers.
inline int32_t element_col(int32_t sb, int32_t reg, int32_t g) {
  return 32 * sb + 16 * (reg >> 3) + 8 * g + (reg & 7);
}

// Validates CSR tile-list structure: ptr[0] == 0, non-decreasing, ptr[n_blocks] == n_tiles,
// columns in range and strictly increasing inside each block.
int check_tile_list(int32_t n_blocks, int32_t n_tiles, int32_t n_cols, const int32_t* ptr,
                    const int32_t* col);

}  // namespace fwn
