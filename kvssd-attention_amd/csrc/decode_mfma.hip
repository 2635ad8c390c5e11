// Matrix-core fused decode kernel (placeholder until the MFMA path lands).
#include "decode.hpp"

namespace kvssd {

bool mfma_supported(const kvssd_decode_desc& d, std::string* why) {
  (void)d;
  if (why) *why = "matrix-core kernel not built";
  return false;
}

MfmaPlan plan_mfma(const kvssd_decode_desc& d, int units) {
  (void)d;
  return MfmaPlan{units, 1, 1};
}

int launch_mfma(const DecodeArgs& a, const MfmaPlan& plan, SplitPartials parts) {
  (void)a;
  (void)plan;
  (void)parts;
  return arg_error("matrix-core kernel not built");
}

}  // namespace kvssd
