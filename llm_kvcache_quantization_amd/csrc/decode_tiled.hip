// Dispatch of the tiled decode kernel (decode_tiled.h): the format family's instantiation,
// looked up in the translation unit that holds it (decode_tiled_{a4,tok,kv4,kv16,kt}.hip), and
// its launch.
#include "decode_common.h"

namespace kvq {

TiledFn tiled_kernel(int fam, int n_rep) {
  const bool pack8 = n_rep <= 8;
  for (auto pick : {tiled_kernel_a4, tiled_kernel_tok, tiled_kernel_kv4, tiled_kernel_kv16,
                    tiled_kernel_kt}) {
    const TiledFn k = pick(fam, pack8);
    if (k.fn) return k;
  }
  return TiledFn{nullptr, nullptr, -1, -1};
}

hipError_t launch_tiled(const DecodeArgs& a, const TiledFn& k, dim3 grid, hipStream_t s) {
  if (!k.fn) return hipErrorInvalidValue;
  DecodeArgs args = a;
  void* kargs[] = {&args};
  return hipLaunchKernel(a.share ? k.fn_share : k.fn, grid, dim3(kTiledWaves * 64), kargs, 0, s);
}

}  // namespace kvq
