// Instantiations of decode_tiled_kernel (decode_tiled.h) for the KIVI-family (4-bit or 8-bit K) families.  The
// families are spread over several translation units so that they compile in parallel.
#include "decode_tiled.h"

namespace kvq {

TiledFn tiled_kernel_kv4(int fam, bool pack8) {
  switch (fam) {
    case kTiledKivi: return tiled_pick<KKiviT, VKiviRowT>(pack8);
    case kTiledKivis: return tiled_pick<KKiviT, VKiviRowTS>(pack8);
    case kTiledKv48: return tiled_pick<KKiviT, VKivi8RowT>(pack8);
    case kTiledKv4F: return tiled_pick<KKiviT, VF16RowT>(pack8);
    case kTiledKv84: return tiled_pick<KKivi8T, VKiviRowT>(pack8);
    case kTiledKv88: return tiled_pick<KKivi8T, VKivi8RowT>(pack8);
    default: return TiledFn{nullptr, nullptr, -1, -1};
  }
}

}  // namespace kvq
