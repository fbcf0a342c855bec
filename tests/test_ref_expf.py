"""ref_expf (wpc-engine_amd/csrc/ref_expf.h), the exp the GPU's softmax and
SiLU use, against the host libm's expf, which is what the reference's
f32::exp calls. Compiled for the host from the same header the HIP kernels
include and compared bit for bit over a strided sweep of all 2^32 bit
patterns (every WPCG_EXPF_STRIDE-th, default 5; stride 1 also passes) plus
the special values. NaN results compare as NaN."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "wpc-engine_amd", "csrc", "ref_expf.h")

HARNESS = r"""
#include "%s"
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
static unsigned long long bad[16], seen[16];
static unsigned long long stride;
static unsigned first[16];
static int same(float a, float b) {
  unsigned ua, ub; memcpy(&ua, &a, 4); memcpy(&ub, &b, 4);
  return ua == ub || (a != a && b != b);
}
static void* run(void* arg) {
  int t = (int)(long)arg;
  for (unsigned long long u = (unsigned long long)t * stride; u < (1ull << 32); u += 16 * stride) {
    unsigned b = (unsigned)u; float x; memcpy(&x, &b, 4);
    seen[t]++;
    if (!same(expf(x), ref_expf(x))) { if (!bad[t]) first[t] = b; bad[t]++; }
  }
  return 0;
}
int main(int argc, char** argv) {
  stride = strtoull(argv[1], 0, 10);
  const float sp[] = {0.0f, -0.0f, 1.0f, -1.0f, 88.0f, -88.0f, 0x1.62e42ep6f, 0x1.62e430p6f,
                      -0x1.9fe368p6f, -0x1.9fe36ap6f, 1e-30f, -1e-30f, 1e30f, -1e30f,
                      __builtin_inff(), -__builtin_inff(), __builtin_nanf("")};
  unsigned long long badsp = 0;
  for (unsigned i = 0; i < sizeof sp / sizeof sp[0]; i++)
    if (!same(expf(sp[i]), ref_expf(sp[i]))) { printf("special %%a: %%a vs %%a\n", sp[i], expf(sp[i]), ref_expf(sp[i])); badsp++; }
  pthread_t th[16];
  for (long i = 0; i < 16; i++) pthread_create(&th[i], 0, run, (void*)i);
  unsigned long long tot = 0, n = 0; unsigned f = 0;
  for (int i = 0; i < 16; i++) { pthread_join(th[i], 0); tot += bad[i]; n += seen[i]; if (bad[i]) f = first[i]; }
  float x; memcpy(&x, &f, 4);
  printf("checked %%llu inputs, %%llu differ", n, tot);
  if (tot) printf(" (e.g. %%a: libm %%a, ref_expf %%a)", x, expf(x), ref_expf(x));
  printf("\n");
  return (tot || badsp) ? 1 : 0;
}
"""


def test_ref_expf_matches_the_host_expf(tmp_path):
    src = tmp_path / "h.c"
    src.write_text(HARNESS % HEADER)
    exe = tmp_path / "h"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm", "-lpthread"],
                   check=True)
    stride = os.environ.get("WPCG_EXPF_STRIDE", "5")
    r = subprocess.run([str(exe), stride], capture_output=True, text=True, timeout=600)
    sys.stdout.write(r.stdout)
    assert r.returncode == 0, r.stdout
