// Instantiations of decode_tiled_kernel (decode_tiled.h) for the INT4_ASYM / static INT8 families.  The
// families are spread over several translation units so that they compile in parallel.
#include "decode_tiled.h"

namespace kvq {

TiledFn tiled_kernel_a4(int fam, bool pack8) {
  switch (fam) {
    case kTiledA4A4: return tiled_pick<KAsymT<false>, VAsymT>(pack8);
    case kTiledA4A4o: return tiled_pick<KAsymT<true>, VAsymT>(pack8);
    case kTiledI8A4: return tiled_pick<KI8T<false>, VAsymT>(pack8);
    case kTiledI8I8: return tiled_pick<KI8T<false>, VI8RowT<false>>(pack8);
    case kTiledI8I8g: return tiled_pick<KI8T<true>, VI8RowT<true>>(pack8);
    default: return TiledFn{nullptr, nullptr, -1, -1};
  }
}

}  // namespace kvq
