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
 */
#include <stdint.h>

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
