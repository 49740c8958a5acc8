// Instantiations of decode_tiled_kernel (decode_tiled.h) for the KIVI-family (8-bit K with fp16 V, fp16 K) and fp16-K / per-token INT8 V families.  The
// families are spread over several translation units so that they compile in parallel.
#include "decode_tiled.h"

namespace kvq {

TiledFn tiled_kernel_kv16(int fam, bool pack8) {
  switch (fam) {
    case kTiledKv8F: return tiled_pick<KKivi8T, VF16RowT>(pack8);
    case kTiledKvF4: return tiled_pick<KF16T, VKiviRowT>(pack8);
    case kTiledKvF8: return tiled_pick<KF16T, VKivi8RowT>(pack8);
    case kTiledKvFF: return tiled_pick<KF16T, VF16RowT>(pack8);
    case kTiledFT8: return tiled_pick<KF16T, VTokT<false>>(pack8);
    default: return TiledFn{nullptr, nullptr, -1, -1};
  }
}

}  // namespace kvq
