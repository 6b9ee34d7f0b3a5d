/*
 * field_oracle.c — TEST INFRASTRUCTURE ONLY. CPU float64 restatement of the Fields LM Field
 * recurrence, used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker of the HIP path. Never part of the product path.
 *
 * It is the textbook sequential first-order linear recurrence, one (b, c) sequence at a time,
 * in double precision, following the reference's CPU path
 *   src/fields_official/reference/field_only_v4_chunked_triton_wiki100.py
 *     reference_field_read  392-416  (gates, complex a/b, displaced readout, output layout)
 *     VAC_MAX               68
 * with the scan of hierarchical_scan/assoc_scan (333-389) replaced by the sequential loop it
 * computes (s_t = a_t s_{t-1} + b_t, s_{-1} = 0). Pinned by tests/test_oracle.py against
 * closed forms (scipy.signal.lfilter, geometric series, T = 1), invariants and the golden
 * fixtures written from the reference itself.
 *
 * Layouts match include/fields_amd.h: raw [B,T,3C], read [B,T,4C], states [B,2C] planar.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

#define FO_VAC_MAX 0.9

static inline double fo_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

/* per-element gates: v, b = gamma*v*inj (reference_field_read, canon:399-406) */
static inline void fo_gates(double zr, double zi, double zv, double gm, double* v, double* br,
                            double* bi) {
  const double inj_r = tanh(zr);
  const double inj_i = tanh(zi);
  const double vac = fo_sigmoid(zv) * FO_VAC_MAX;
  *v = vac;
  *br = gm * vac * inj_r;
  *bi = gm * vac * inj_i;
}

/*
 * Full-sequence scan. raw row (b,t) starts at raw + b*sb + t*st. state_in/state_out may be NULL.
 */
void fo_scan_f64(const double* raw, int64_t B, int64_t T, int64_t C, int64_t sb, int64_t st,
                 const double* tr, const double* ti, const double* gamma,
                 const double* state_in, double* state_out, double* read) {
  for (int64_t b = 0; b < B; ++b) {
    for (int64_t c = 0; c < C; ++c) {
      double sr = state_in ? state_in[b * 2 * C + c] : 0.0;
      double si = state_in ? state_in[b * 2 * C + C + c] : 0.0;
      const double lr = tr[c], li = ti[c], gm = gamma[c];
      for (int64_t t = 0; t < T; ++t) {
        const double* z = raw + b * sb + t * st;
        double v, br, bi;
        fo_gates(z[c], z[C + c], z[2 * C + c], gm, &v, &br, &bi);
        /* moved = lam * s_{t-1}; displaced = v * moved (canon:408-410) */
        const double mr = lr * sr - li * si;
        const double mi = lr * si + li * sr;
        const double dr = v * mr;
        const double di = v * mi;
        /* a = (1 - v) * lam; s_t = a * s_{t-1} + b (canon:404-407) */
        const double ar = (1.0 - v) * lr;
        const double ai = (1.0 - v) * li;
        const double nr = ar * sr - ai * si + br;
        const double ni = ar * si + ai * sr + bi;
        sr = nr;
        si = ni;
        double* o = read + (b * T + t) * 4 * C;
        o[c] = sr;
        o[C + c] = si;
        o[2 * C + c] = dr;
        o[3 * C + c] = di;
      }
      if (state_out) {
        state_out[b * 2 * C + c] = sr;
        state_out[b * 2 * C + C + c] = si;
      }
    }
  }
}

/* One decode step: state (planar [B,2C]) updated in place, read_t [B,4C] written. */
void fo_decode_step_f64(const double* raw_t, int64_t B, int64_t C, int64_t sb, const double* tr,
                        const double* ti, const double* gamma, double* state, double* read_t) {
  for (int64_t b = 0; b < B; ++b) {
    const double* z = raw_t + b * sb;
    for (int64_t c = 0; c < C; ++c) {
      double v, br, bi;
      fo_gates(z[c], z[C + c], z[2 * C + c], gamma[c], &v, &br, &bi);
      const double sr = state[b * 2 * C + c], si = state[b * 2 * C + C + c];
      const double mr = tr[c] * sr - ti[c] * si;
      const double mi = tr[c] * si + ti[c] * sr;
      const double ar = (1.0 - v) * tr[c], ai = (1.0 - v) * ti[c];
      const double nr = ar * sr - ai * si + br;
      const double ni = ar * si + ai * sr + bi;
      state[b * 2 * C + c] = nr;
      state[b * 2 * C + C + c] = ni;
      double* o = read_t + b * 4 * C;
      o[c] = nr;
      o[C + c] = ni;
      o[2 * C + c] = v * mr;
      o[3 * C + c] = v * mi;
    }
  }
}
