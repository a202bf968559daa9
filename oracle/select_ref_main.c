/*
 * Command-line driver of oracle/select_ref.c, for the sanitizer build.
 *
 * TEST INFRASTRUCTURE ONLY (built by `make -C oracle asan`, run by
 * tests/test_oracle.py): reads two fp32 score files of [BH, S_tot] rows, runs
 * lh_ref_select and writes the int32 [BH, out_len] result, so that the
 * restatement can run under AddressSanitizer and UndefinedBehaviorSanitizer in
 * a process of its own.
 *
 *   select_ref_asan BH S_tot S L p topk tie_lower mode out_len qk.f32 kq.f32 out.i32
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

int lh_ref_select(const float *scores_qk, const float *scores_kq, int BH, int S_tot,
                  int S, int L, int p, int topk, int tie_lower, int mode,
                  int32_t *out, int out_len);

static int read_all(const char *path, void *buf, size_t bytes) {
  FILE *f = fopen(path, "rb");
  if (!f) return -1;
  size_t got = fread(buf, 1, bytes, f);
  fclose(f);
  return got == bytes ? 0 : -1;
}

int main(int argc, char **argv) {
  if (argc != 13) {
    fprintf(stderr, "usage: %s BH S_tot S L p topk tie_lower mode out_len qk kq out\n", argv[0]);
    return 2;
  }
  int a[9];
  for (int i = 0; i < 9; ++i) a[i] = atoi(argv[1 + i]);
  const int BH = a[0], S_tot = a[1], out_len = a[8];
  if (BH <= 0 || S_tot <= 0 || out_len <= 0) return 2;
  const size_t n_in = (size_t)BH * S_tot, n_out = (size_t)BH * out_len;
  float *qk = malloc(n_in * sizeof(float)), *kq = malloc(n_in * sizeof(float));
  int32_t *out = malloc(n_out * sizeof(int32_t));
  if (!qk || !kq || !out) return 3;
  if (read_all(argv[10], qk, n_in * sizeof(float)) || read_all(argv[11], kq, n_in * sizeof(float))) return 4;
  int rc = lh_ref_select(qk, kq, BH, S_tot, a[2], a[3], a[4], a[5], a[6], a[7], out, out_len);
  if (rc == 0) {
    FILE *f = fopen(argv[12], "wb");
    if (!f || fwrite(out, sizeof(int32_t), n_out, f) != n_out) rc = 5;
    if (f) fclose(f);
  }
  free(qk); free(kq); free(out);
  return rc < 0 ? 10 - rc : rc;
}
