/* Test infrastructure: compares eg2_f32_to_chars (libeg2hip.so) with the
 * reference's ei_f32_to_chars (vendor/embeddinggemma.c/src/float_format.c,
 * compiled into _ref/libref.so) byte for byte over every stride-th float
 * bit pattern, on several threads. Prints the patterns compared and the
 * mismatches (the first few in full); exits 1 on any mismatch.
 *   float_text_check <stride> [threads] [libref.so] [libeg2hip.so] */
#include <dlfcn.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef size_t (*fmt_fn)(char *, float);
static fmt_fn ref_fmt, our_fmt;
static uint64_t stride = 1;
static unsigned threads = 8;
static uint64_t mismatches, compared;
static pthread_mutex_t lock = PTHREAD_MUTEX_INITIALIZER;

static void *run(void *arg) {
  const unsigned id = (unsigned)(uintptr_t)arg;
  uint64_t bad = 0, seen = 0;
  for (uint64_t i = (uint64_t)id * stride; i < (1ull << 32); i += (uint64_t)threads * stride) {
    const uint32_t bits = (uint32_t)i;
    float v;
    memcpy(&v, &bits, 4);
    char a[64], b[64];
    const size_t na = ref_fmt(a, v), nb = our_fmt(b, v);
    ++seen;
    if (na != nb || memcmp(a, b, na) != 0) {
      if (bad++ < 5) {
        pthread_mutex_lock(&lock);
        fprintf(stderr, "0x%08x: reference %.*s, ours %.*s\n", bits, (int)na, a, (int)nb, b);
        pthread_mutex_unlock(&lock);
      }
    }
  }
  pthread_mutex_lock(&lock);
  mismatches += bad;
  compared += seen;
  pthread_mutex_unlock(&lock);
  return NULL;
}

int main(int argc, char **argv) {
  if (argc > 1) stride = strtoull(argv[1], NULL, 10);
  if (argc > 2) threads = (unsigned)strtoul(argv[2], NULL, 10);
  const char *ref_path = argc > 3 ? argv[3] : "_ref/libref.so";
  const char *our_path = argc > 4 ? argv[4] : "../embeddinggemma2-amdkfd_amd/libeg2hip.so";
  if (stride == 0 || threads == 0 || threads > 256) return 2;
  void *r = dlopen(ref_path, RTLD_NOW | RTLD_LOCAL), *o = dlopen(our_path, RTLD_NOW | RTLD_LOCAL);
  if (!r || !o) {
    fprintf(stderr, "dlopen: %s\n", dlerror());
    return 2;
  }
  ref_fmt = (fmt_fn)dlsym(r, "ei_f32_to_chars");
  our_fmt = (fmt_fn)dlsym(o, "eg2_f32_to_chars");
  if (!ref_fmt || !our_fmt) {
    fprintf(stderr, "missing symbol: %s\n", !ref_fmt ? "ei_f32_to_chars" : "eg2_f32_to_chars");
    return 2;
  }
  pthread_t t[256];
  for (unsigned i = 0; i < threads; ++i) pthread_create(&t[i], NULL, run, (void *)(uintptr_t)i);
  for (unsigned i = 0; i < threads; ++i) pthread_join(t[i], NULL);
  printf("compared %llu bit patterns (stride %llu), %llu mismatches\n", (unsigned long long)compared,
         (unsigned long long)stride, (unsigned long long)mismatches);
  return mismatches ? 1 : 0;
}
