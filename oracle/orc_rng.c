/*
 * orc_rng.c - seeded synthetic inputs shared by the CPU oracle, the golden
 * generator and (restated in HIP) the device fill used by bench.py.
 * TEST INFRASTRUCTURE ONLY (see orc.h).
 *
 * SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
 * generators", OOPSLA 2014): state += golden gamma, then the variant-13
 * finaliser.  Uniform doubles use the top 53 bits, shifted into (0,1] so
 * that log() is finite.  Normals use the Box-Muller transform in double:
 * a pair (u1,u2) gives r*cos(2*pi*u2) then r*sin(2*pi*u2), r = sqrt(-2 ln u1),
 * each rounded to float.  Element i of a stream therefore depends only on
 * outputs 2*(i/2) and 2*(i/2)+1 of the generator, which lets the device
 * compute any element from its index.
 */
#define _POSIX_C_SOURCE 199309L
#include "orc.h"
#include <math.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_GAMMA 0x9e3779b97f4a7c15ull

static uint64_t orc_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t orc_splitmix64(uint64_t *state) {
  *state += ORC_GAMMA;
  return orc_mix64(*state);
}

double orc_uniform01(uint64_t *state) {
  uint64_t z = orc_splitmix64(state);
  return (double)((z >> 11) + 1ull) * (1.0 / 9007199254740992.0);
}

void orc_normal_f32(uint64_t *state, float *out, size_t n) {
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = orc_uniform01(state);
    double u2 = orc_uniform01(state);
    double r = sqrt(-2.0 * log(u1));
    double a = two_pi * u2;
    out[i++] = (float)(r * cos(a));
    if (i < n) out[i++] = (float)(r * sin(a));
  }
}

double orc_now_sec(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

int orc_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
