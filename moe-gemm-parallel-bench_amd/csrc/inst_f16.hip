// Compiled f16 tile configurations.
#include "registry.h"
namespace moegemm {
MOEGEMM_MENU_16BIT(MOEGEMM_INST16, EF16)
#if !defined(__HIP_DEVICE_COMPILE__)
MOEGEMM_MENU_16BIT(MOEGEMM_EXTERN16_SK, EF16)
const KernelEntry kEntriesF16[] = {MOEGEMM_MENU_16BIT(MOEGEMM_ENTRY16, EF16)};
const int kNumF16 = sizeof(kEntriesF16) / sizeof(kEntriesF16[0]);
#endif
}  // namespace moegemm
