// Compiled f32 tile configurations.
#include "registry.h"
namespace moegemm {
MOEGEMM_MENU_F32(MOEGEMM_INST32, EF32)
#if !defined(__HIP_DEVICE_COMPILE__)
const KernelEntry kEntriesF32[] = {MOEGEMM_MENU_F32(MOEGEMM_ENTRY32, EF32)};
const int kNumF32 = sizeof(kEntriesF32) / sizeof(kEntriesF32[0]);
#endif
}  // namespace moegemm
