// Instantiations of decode_tiled_kernel (decode_tiled.h) for the per-token asymmetric INT4 K
// families (KTokAsymT).  The families are spread over several translation units so that they
// compile in parallel.
#include "decode_tiled.h"

namespace kvq {

TiledFn tiled_kernel_kt(int fam, bool pack8) {
  switch (fam) {
    case kTiledKtKv: return tiled_pick<KTokAsymT, VKiviRowT>(pack8);
    case kTiledKtT8: return tiled_pick<KTokAsymT, VTokT<false>>(pack8);
    case kTiledKtF: return tiled_pick<KTokAsymT, VF16RowT>(pack8);
    default: return TiledFn{nullptr, nullptr, -1, -1};
  }
}

}  // namespace kvq
