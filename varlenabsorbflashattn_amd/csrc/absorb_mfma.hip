// Absorbed target attention on gfx950 matrix cores (bf16 / f16 inputs).
#include "kernels.h"
#include "mfma.h"

namespace vafa {

template <typename T>
bool mfma_absorb_supported(int H, int F, int DH) {
  (void)H;
  (void)F;
  (void)DH;
  return false;
}

template <typename T>
void launch_mfma_absorb_fwd(const AbsorbArgs &, hipStream_t) {}

template bool mfma_absorb_supported<bf16>(int, int, int);
template bool mfma_absorb_supported<f16>(int, int, int);
template void launch_mfma_absorb_fwd<bf16>(const AbsorbArgs &, hipStream_t);
template void launch_mfma_absorb_fwd<f16>(const AbsorbArgs &, hipStream_t);

}  // namespace vafa
