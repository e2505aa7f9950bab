// Host-only driver for tests/test_host_sanitizers.py: exercises the C ABI's
// host logic (tables, planner, argument checks, context creation without a
// device) under AddressSanitizer and UndefinedBehaviorSanitizer.  Returns
// the number of failed checks.
#include <cstdio>
#include <cstdlib>
#include <vector>
#include "scriptrs_fe.h"
int main() {
  sfe_config c; sfe_config_default(&c);
  std::vector<float> win(400), fb(128 * 257);
  if (sfe_build_tables(&c, win.data(), fb.data())) return 1;
  sfe_overlap_config oc; sfe_overlap_config_default(&oc);
  long total = 0;
  for (int64_t len : {0LL, 1LL, 1279LL, 1280LL, 238080LL, 238081LL, 57600000LL, 460800000LL}) {
    int32_t n = 0;
    int rc = sfe_plan_fast(&oc, len, nullptr, 0, &n);
    std::vector<sfe_chunk> t(n > 0 ? n : 1);
    rc = sfe_plan_fast(&oc, len, t.data(), n, &n);
    total += n;
    if (rc && len > 0) { printf("plan rc %d len %lld\n", rc, (long long)len); return 1; }
  }
  for (double ov : {-1.0, 0.0, 0.5, 2.0, 1e30}) {
    sfe_overlap_config o2 = oc; o2.overlap_seconds = ov; int32_t n = 0;
    std::vector<sfe_chunk> t(4096);
    sfe_plan_fast(&o2, 1000000, t.data(), 4096, &n);
  }
  // argument errors before any device work
  float buf[1024] = {0}; int64_t fo[3]; sfe_chunk tk[1] = {{0, 100, 0, 0}};
  int bad = 0;
  bad += sfe_extract(nullptr, buf, 0, buf, 0) != SFE_EMPTY_AUDIO;
  bad += sfe_extract_chunks_pcm(nullptr, buf, 7, 16, 1000, tk, 1, 0, buf, fo, nullptr) != SFE_INVALID_ARG;
  bad += sfe_extract_chunks_pcm(nullptr, buf, 1, 1, 1000, tk, 1, 0, buf, fo, nullptr) != SFE_INVALID_ARG;
  bad += sfe_extract_chunks(nullptr, buf, 10, tk, 1, 0, buf, fo, nullptr) != SFE_INVALID_ARG;
  bad += sfe_extract_chunks(nullptr, buf, 1000, tk, 1, 9, buf, fo, nullptr) != SFE_INVALID_ARG;
  bad += sfe_vad_frames(nullptr, buf, 0, 32, -1, buf, 1, nullptr) != SFE_INVALID_ARG;
  bad += sfe_vad_frames(nullptr, buf, 0, 32, 2000, buf, 1, nullptr) != SFE_INVALID_ARG;
  bad += sfe_vad_num_windows(513) != 2;
  sfe_ctx* ctx = nullptr;
  int rc = sfe_create(&c, 0, &ctx);  // no GPU here: an error, no leak
  printf("create rc %d (%s)\n", rc, sfe_last_error());
  printf("tasks %ld bad %d\n", total, bad);
  return bad;
}
