// Instantiations of decode_tiled_kernel (decode_tiled.h) for the per-token scale families.  The
// families are spread over several translation units so that they compile in parallel.
#include "decode_tiled.h"

namespace kvq {

TiledFn tiled_kernel_tok(int fam, bool pack8) {
  switch (fam) {
    case kTiledT8: return tiled_pick<KTokT<false, 1>, VTokT<false>>(pack8);
    case kTiledT8g16: return tiled_pick<KTokT<false, 2>, VTokT<false>>(pack8);
    case kTiledT4: return tiled_pick<KTokT<true, 1>, VTokT<true>>(pack8);
    case kTiledT4g16: return tiled_pick<KTokT<true, 2>, VTokT<true>>(pack8);
    case kTiledT4s: return tiled_pick<KTokT<true, 1>, VTokT<true, true>>(pack8);
    case kTiledT4g16s: return tiled_pick<KTokT<true, 2>, VTokT<true, true>>(pack8);
    case kTiledT8Kv: return tiled_pick<KTokT<false, 1>, VKiviRowT>(pack8);
    case kTiledT8Kvg16: return tiled_pick<KTokT<false, 2>, VKiviRowT>(pack8);
    case kTiledT8Kvs: return tiled_pick<KTokT<false, 1>, VKiviRowTS>(pack8);
    case kTiledT8Kvg16s: return tiled_pick<KTokT<false, 2>, VKiviRowTS>(pack8);
    case kTiledT8F: return tiled_pick<KTokT<false, 1>, VF16RowT>(pack8);
    case kTiledT8Fg16: return tiled_pick<KTokT<false, 2>, VF16RowT>(pack8);
    default: return TiledFn{nullptr, nullptr, -1, -1};
  }
}

}  // namespace kvq
