// Compiled f16 stream-K kernels (a unit of their own: see MOEGEMM_INST16_SK in registry.h).
#include "registry.h"
namespace moegemm {
MOEGEMM_MENU_16BIT(MOEGEMM_INST16_SK, EF16)
}  // namespace moegemm
