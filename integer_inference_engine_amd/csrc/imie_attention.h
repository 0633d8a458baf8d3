// Attention problem descriptor shared by the attention kernels and the layer pipelines.
#pragma once
#include "imie_common.h"

struct AttnDesc {
  int64_t B, H, Hkv, hd, M;        // query rows (b, h, m): q[b*qsb + h*qsh + m*qsm + c]
  int64_t qsb, qsh, qsm;           // element strides of q and out (out uses the same strides)
  const int64_t* q;
  const void* K;                   // paged pools (see attention.hip)
  const void* V;
  int kv32;                        // 1: kv8 digit-plane cache (imie_kvfmt.h), 0: int64 elements
  const uint64_t *run_k, *run_v;   // kv8: running max|K|, max|V| per (sequence, kv head) [B*Hkv]
  const int8_t* qd;                // kv8 decode (optional): q digit planes [B*H][8][hd] from the head stage
  const int* qlimbs;               //   and their limb counts [B*H] (maxq then points at the head stage's max|q|)
  const int64_t* pt;               // page table [B][mp]
  int64_t P, mp;                   // tokens per page, pages per sequence
  int pshift;                      // log2(P) when P is a power of two, else -1 (set by the launcher)
  const int64_t* lengths;          // decode: keys per sequence (starts == nullptr)
  const int64_t* starts;           // causal: first new position per sequence (M new rows)
  int64_t Lmax;                    // score row stride (>= max visible keys)
  int frac;
  int64_t inv_sqrt, log2e, dclip;
  int64_t* out;
  int* status;
  const uint64_t* rope_guard;      // optional: q/k RoPE envelope maxima (4 x u64), checked by the final kernel
  // scratch (imie_attn_bind_scratch)
  int64_t* scores;
  uint64_t* acc;
  int64_t* rowmax;
  uint64_t *maxq, *maxp, *maxk, *maxv;
  uint64_t* part;                  // decode: per-chunk PV partials [nch][B*H][hd]
  int64_t* cmax;                   // decode: per-chunk row max of the scores [nch][B*H]
  uint64_t *cz, *cmp;              // decode: per-chunk Z and max p [nch][B*H]
  uint64_t *ckm, *cvm;             // decode: per-chunk max|K|, max|V| [nch][B*Hkv]
  int64_t chunk, nch;              // decode key chunking (set by the launcher)
  int64_t* pmax;                   // prefill kv8: per-256-key row maxima [nkt][rows]
  int8_t* pd;                      // prefill kv8: digit planes of p [4][rows][pdL]
  int64_t pdL;                     // row stride of pd (Lmax rounded up to 16)
};

size_t imie_attn_scratch_bytes(int64_t B, int64_t H, int64_t Hkv, int64_t M, int64_t hd, int64_t Lmax);
// Decode (M == 1) only: the q digit-plane buffer and limb counts inside bound scratch, for a head stage that
// prepares them (then set d.qd, d.qlimbs and point d.maxq at the head stage's max|q|)
void imie_attn_qdigit_scratch(const AttnDesc& d, int8_t** qd, int** qlimbs);
void imie_attn_bind_scratch(AttnDesc& d, void* scratch);
int imie_attention_launch(AttnDesc d, hipStream_t st);
