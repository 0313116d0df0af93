// Mamba-2 SSD chunk scan backward for gfx950 (see ssd.hip for the forward).
#include "common.hpp"
#include "io.hpp"
#include "mma.hpp"
#include "ssd.hpp"

using namespace mko;
using namespace mko::ssd;

extern "C" size_t mko_ssd_bwd_workspace_size(const mko_ssd_params* prm) {
  Geo g;
  if (make_geo(prm, &g) != MKO_OK) return 0;
  return 0;
}

extern "C" int mko_ssd_bwd(const mko_ssd_params* prm, void* stream) {
  (void)prm;
  (void)stream;
  mko_set_error("ssd_bwd: not built yet");
  return MKO_EUNSUPPORTED;
}
