// Compiled bf16 tile configurations.
#include "registry.h"
namespace moegemm {
MOEGEMM_MENU_16BIT(MOEGEMM_INST16, EBf16)
#if !defined(__HIP_DEVICE_COMPILE__)
MOEGEMM_MENU_16BIT(MOEGEMM_EXTERN16_SK, EBf16)
const KernelEntry kEntriesBf16[] = {MOEGEMM_MENU_16BIT(MOEGEMM_ENTRY16, EBf16)};
const int kNumBf16 = sizeof(kEntriesBf16) / sizeof(kEntriesBf16[0]);
#endif
}  // namespace moegemm
