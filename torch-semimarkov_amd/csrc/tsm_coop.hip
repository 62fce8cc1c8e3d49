// Cooperative scan instances (tsm_coopscan.hpp), log and max-plus semirings: 16
// lanes per label, eight source labels per lane in the label mix (C <= 128),
// durations per lane in steps of 8 (padded durations carry a -1e30 duration bias).
#include "tsm_coopscan.hpp"

namespace tsm {

namespace {

template <int R, bool LOGSR>
int launch_coop_r(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  return fwd ? coop::launch_coop_dir<coop::CoopChunk<16, R, 8, true, LOGSR>>(pl, p, st)
             : coop::launch_coop_dir<coop::CoopChunk<16, R, 8, false, LOGSR>>(pl, p, st);
}

template <bool LOGSR>
int launch_coop_sr(const Plan& pl, const ScanParams& p, bool forward, hipStream_t st) {
  switch (pl.CR) {
    case 8: return launch_coop_r<8, LOGSR>(pl, p, forward, st);
    case 16: return launch_coop_r<16, LOGSR>(pl, p, forward, st);
    case 24: return launch_coop_r<24, LOGSR>(pl, p, forward, st);
    case 32: return launch_coop_r<32, LOGSR>(pl, p, forward, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace

int launch_coop_scan(const Plan& pl, const ScanParams& p, bool forward, bool logsr, hipStream_t st) {
  return logsr ? launch_coop_sr<true>(pl, p, forward, st) : launch_coop_sr<false>(pl, p, forward, st);
}

}  // namespace tsm
