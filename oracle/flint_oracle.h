/* flint_oracle.h -- CPU restatement of the Flint KV path (TEST INFRASTRUCTURE ONLY; see flint_oracle.c). */
#ifndef FLINT_ORACLE_H
#define FLINT_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

void orc_fl_rope_table(int pos, float base, float* tab);
void orc_fl_rope(int ntok, int heads, const float* x, const float* tab, float* out);
void orc_fl_kv_write(int fmt, void* kc, void* vc, int ring, int pos0, int n, const float* k, const float* v);
void orc_fl_attn_fd(int fmt, const void* kc, const void* vc, int ring, const float* q, int lo, int n,
                    const float* sinks, float* out);
void orc_fl_attn_pf(int fmt, const void* kc, const void* vc, int ring, const float* q, int pos0, int n, int win,
                    const float* sinks, float* out);

#ifdef __cplusplus
}
#endif
#endif
