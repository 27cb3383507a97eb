/*
 * CPU oracle (TEST INFRASTRUCTURE ONLY -- never linked into the product) for
 * the radius graph of mlcg's SchNet neighbour list.
 *
 * Restates, for every frame independently, the brute-force search of the
 * reference's native kernel: src/opt_radius/mlcg_opt_radius/radius.cu:117-141
 * (loop over all nodes of the frame in ascending index, squared distance
 * accumulated as 0 + dx*dx + dy*dy + dz*dz, strict `dist < r` with r = r*r
 * computed in double on the host and cast to the scalar type at line 250,
 * optional self-loop skip, rows truncated to their first max_num_neighbors
 * hits).  Output is the canonical edge list: rows (centre i) ascending,
 * neighbours j ascending.
 *
 * Optional exclusions restate the reference's merge walk over the centre's
 * sorted exclusion segment (radius.cu:30-58 is_in_sorted_array, called for
 * every candidate at 113-133): the cursor advances past smaller values and a
 * candidate is excluded when the cursor value equals it.  Excluded candidates
 * do not count towards max_num_neighbors.
 *
 * Built with -ffp-contract=off so that every product and sum is rounded to
 * float separately (no FMA), which is the arithmetic the HIP kernel uses.
 *
 * float16 / bfloat16 positions (the reference's Half / BFloat16 dispatch,
 * radius.cu:243-250) follow the c10 scalar arithmetic: every operator converts
 * its operands to float, operates, and rounds the result back to the 16-bit
 * type (round to nearest, ties to even); r*r is computed in double, rounded
 * to float, then to the 16-bit type; the comparison is made in float.  The
 * conversions below are written from the IEEE 754 binary16 and the bfloat16
 * (truncated binary32) formats.
 */
#include <stdint.h>
#include <string.h>

/* radius.cu:30-58: advances *cur over xs[*cur, end) while below q. */
static int merge_member(int64_t q, const int64_t* xs, int64_t* cur, int64_t end) {
  while (*cur < end) {
    int64_t v = xs[*cur];
    if (v < q)
      ++*cur;
    else
      return v == q;
  }
  return 0;
}

static float sqdist(const float* pos, int64_t i, int64_t j) {
  float dx = pos[3 * j + 0] - pos[3 * i + 0];
  float dy = pos[3 * j + 1] - pos[3 * i + 1];
  float dz = pos[3 * j + 2] - pos[3 * i + 2];
  float s = dx * dx;
  s = s + dy * dy;
  s = s + dz * dz;
  return s;
}

/* deg[i] for every node; returns the total edge count, -1 on bad input.
 * *overflow is set when some row had more than max_nn hits. */
int64_t oracle_radius_count(const float* pos, const int64_t* frame_ptr, int64_t n_frames,
                            double r, int loop, int64_t max_nn, const int64_t* exs,
                            const int64_t* eptr, int64_t* deg, int* overflow) {
  const float r2 = (float)(r * r);
  int64_t total = 0;
  *overflow = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0, hits = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1]; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist(pos, i, j) < r2) {
          ++hits;
          if (c < max_nn) ++c;
        }
      }
      if (hits > max_nn) *overflow = 1;
      deg[i] = c;
      total += c;
    }
  }
  return total;
}

/* Writes edges into ei0 (centre) / ei1 (neighbour), each of length
 * sum(deg). */
void oracle_radius_fill(const float* pos, const int64_t* frame_ptr, int64_t n_frames,
                        double r, int loop, int64_t max_nn, const int64_t* exs,
                        const int64_t* eptr, int64_t* ei0, int64_t* ei1) {
  const float r2 = (float)(r * r);
  int64_t e = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1] && c < max_nn; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist(pos, i, j) < r2) {
          ei0[e] = i;
          ei1[e] = j;
          ++e;
          ++c;
        }
      }
    }
  }
}

/* The same search for float64 positions: d2 in double, d2 < r*r
 * (radius.cu's scalar_t = double instantiation). */
static double sqdist_f64(const double* pos, int64_t i, int64_t j) {
  double dx = pos[3 * j + 0] - pos[3 * i + 0];
  double dy = pos[3 * j + 1] - pos[3 * i + 1];
  double dz = pos[3 * j + 2] - pos[3 * i + 2];
  double s = dx * dx;
  s = s + dy * dy;
  s = s + dz * dz;
  return s;
}

/* deg[i] for every node; returns the total edge count, -1 on bad input.
 * *overflow is set when some row had more than max_nn hits. */
int64_t oracle_radius_count_f64(const double* pos, const int64_t* frame_ptr, int64_t n_frames,
                            double r, int loop, int64_t max_nn, const int64_t* exs,
                            const int64_t* eptr, int64_t* deg, int* overflow) {
  const double r2 = r * r;
  int64_t total = 0;
  *overflow = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0, hits = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1]; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist_f64(pos, i, j) < r2) {
          ++hits;
          if (c < max_nn) ++c;
        }
      }
      if (hits > max_nn) *overflow = 1;
      deg[i] = c;
      total += c;
    }
  }
  return total;
}

/* Writes edges into ei0 (centre) / ei1 (neighbour), each of length
 * sum(deg). */
void oracle_radius_fill_f64(const double* pos, const int64_t* frame_ptr, int64_t n_frames,
                        double r, int loop, int64_t max_nn, const int64_t* exs,
                        const int64_t* eptr, int64_t* ei0, int64_t* ei1) {
  const double r2 = r * r;
  int64_t e = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1] && c < max_nn; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist_f64(pos, i, j) < r2) {
          ei0[e] = i;
          ei1[e] = j;
          ++e;
          ++c;
        }
      }
    }
  }
}

/* ---- 16-bit position types ------------------------------------------- */

static float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* binary16 -> float (exact). */
static float h16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1f) return bits_to_f32(sign | 0x7f800000u | (m << 13)); /* inf / nan */
  if (e == 0) { /* zero or subnormal: m * 2^-24 */
    float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* float -> binary16, round to nearest, ties to even. */
static uint16_t f32_to_h16(float f) {
  const uint32_t u = f32_to_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* nan */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520: rounds to inf */
  if (a < 0x38800000u) { /* below 2^-14: subnormal result, units of 2^-24 */
    /* |f| * 2^24 rounded to an integer, ties to even; exact in float for
     * |f| < 2^-14 since the product only moves the exponent */
    const float scaled = bits_to_f32(a) * 16777216.0f;
    float r = (float)(uint32_t)scaled;
    const float frac = scaled - r;
    if (frac > 0.5f || (frac == 0.5f && ((uint32_t)r & 1u))) r += 1.0f;
    return (uint16_t)(sign | (uint16_t)(uint32_t)r);
  }
  /* normal: keep 10 of the 23 fraction bits, round on the 13 dropped ones */
  const uint32_t e = (a >> 23) - 112u, m = a & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  const uint32_t rest = m & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u; /* may carry into e */
  return (uint16_t)(sign | h);
}

/* bfloat16 -> float (exact). */
static float b16_to_f32(uint16_t b) { return bits_to_f32((uint32_t)b << 16); }

/* float -> bfloat16, round to nearest, ties to even. */
static uint16_t f32_to_b16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* nan */
  const uint32_t rest = u & 0xffffu;
  uint32_t hi = u >> 16;
  if (rest > 0x8000u || (rest == 0x8000u && (hi & 1u))) hi += 1u;
  return (uint16_t)hi;
}

/* kind 0: binary16, kind 1: bfloat16.  One operation: float, then rounded. */
static float narrow_round(int kind, float v) {
  return kind ? b16_to_f32(f32_to_b16(v)) : h16_to_f32(f32_to_h16(v));
}

static float narrow_load(int kind, const uint16_t* pos, int64_t k) {
  return kind ? b16_to_f32(pos[k]) : h16_to_f32(pos[k]);
}

static float sqdist_narrow(int kind, const uint16_t* pos, int64_t i, int64_t j) {
  const float dx = narrow_round(kind, narrow_load(kind, pos, 3 * j) - narrow_load(kind, pos, 3 * i));
  const float dy = narrow_round(kind, narrow_load(kind, pos, 3 * j + 1) -
                                          narrow_load(kind, pos, 3 * i + 1));
  const float dz = narrow_round(kind, narrow_load(kind, pos, 3 * j + 2) -
                                          narrow_load(kind, pos, 3 * i + 2));
  float s = narrow_round(kind, dx * dx);
  s = narrow_round(kind, s + narrow_round(kind, dy * dy));
  s = narrow_round(kind, s + narrow_round(kind, dz * dz));
  return s;
}

/* Exposed for the oracle's own tests: the two conversions. */
uint16_t oracle_f32_to_narrow(int kind, float f) { return kind ? f32_to_b16(f) : f32_to_h16(f); }
float oracle_narrow_to_f32(int kind, uint16_t b) { return kind ? b16_to_f32(b) : h16_to_f32(b); }

int64_t oracle_radius_count_n16(int kind, const uint16_t* pos, const int64_t* frame_ptr,
                                int64_t n_frames, double r, int loop, int64_t max_nn,
                                const int64_t* exs, const int64_t* eptr, int64_t* deg,
                                int* overflow) {
  const float r2 = narrow_round(kind, (float)(r * r));
  int64_t total = 0;
  *overflow = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0, hits = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1]; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist_narrow(kind, pos, i, j) < r2) {
          ++hits;
          if (c < max_nn) ++c;
        }
      }
      if (hits > max_nn) *overflow = 1;
      deg[i] = c;
      total += c;
    }
  }
  return total;
}

void oracle_radius_fill_n16(int kind, const uint16_t* pos, const int64_t* frame_ptr,
                            int64_t n_frames, double r, int loop, int64_t max_nn,
                            const int64_t* exs, const int64_t* eptr, int64_t* ei0,
                            int64_t* ei1) {
  const float r2 = narrow_round(kind, (float)(r * r));
  int64_t e = 0;
  for (int64_t b = 0; b < n_frames; ++b) {
    for (int64_t i = frame_ptr[b]; i < frame_ptr[b + 1]; ++i) {
      int64_t c = 0;
      int64_t cur = exs ? eptr[i] : 0, end = exs ? eptr[i + 1] : 0;
      for (int64_t j = frame_ptr[b]; j < frame_ptr[b + 1] && c < max_nn; ++j) {
        int excluded = exs ? merge_member(j, exs, &cur, end) : 0;
        if (excluded || (!loop && j == i)) continue;
        if (sqdist_narrow(kind, pos, i, j) < r2) {
          ei0[e] = i;
          ei1[e] = j;
          ++e;
          ++c;
        }
      }
    }
  }
}
