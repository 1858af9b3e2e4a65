// hy3x_mfma_wide.hip -- the wide shape of the MFMA grouped GEMMs (64-token
// tiles, 8 waves per workgroup): the same source as the narrow shape,
// compiled with HY3X_MFMA_WIDE into namespace hy3x::mfma_wide.
#define HY3X_MFMA_WIDE
#include "hy3x_mfma.hip"
