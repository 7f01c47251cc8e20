// ref_fa_shim.cpp -- builds the reference flash-attention runners' CPU-side
// code, from the reference checkout, into oracle/_ref/libref_fa_*.so.
//
// TEST INFRASTRUCTURE ONLY.  The runner source is pulled in with -include on
// the compile line (oracle/Makefile); its `main` is renamed by -Dmain=... so
// the shared object only exposes the C entry points below.  Which runner is
// included is chosen by REF_FA_GFX950 (wave-fa-gfx950-runner.cpp) or not
// (wave-fa-calibrate-runner.cpp).
#include <cstdint>
#include <cstring>

extern "C" {

#ifdef REF_FA_GFX950
// makeInput (wave-fa-gfx950-runner.cpp:194-202)
void ref_fa_gfx950_make_input(size_t count, int seed, int stream, float scale,
                              uint16_t *out) {
  std::vector<uint16_t> v = makeInput(count, seed, stream, scale);
  std::memcpy(out, v.data(), count * sizeof(uint16_t));
}

// computeAttentionRow (:247-279) for one (head, row) of a B*H*S*128 problem.
void ref_fa_gfx950_attention_row(int batch, int heads, int sequence,
                                 const uint16_t *q, const uint16_t *k,
                                 const uint16_t *v, int head, int row,
                                 float *out) {
  Args args;
  args.batch = batch;
  args.heads = heads;
  args.sequence = sequence;
  size_t n = static_cast<size_t>(batch) * heads * sequence * kHeadDim;
  std::vector<uint16_t> qv(q, q + n), kv(k, k + n), vv(v, v + n);
  ReferenceRow r = computeAttentionRow(args, qv, kv, vv, head, row);
  std::memcpy(out, r.values.data(), kHeadDim * sizeof(float));
}
#else
// makeInputs + computeReference (wave-fa-calibrate-runner.cpp:197-249)
void ref_fa_f32_inputs_and_reference(int block_m, int seq_n, int head_dim,
                                     int seed, uint16_t *q, uint16_t *k,
                                     uint16_t *v, float *out) {
  Args a;
  a.blockM = block_m;
  a.seqN = seq_n;
  a.headDim = head_dim;
  a.seed = seed;
  std::vector<float> hq(static_cast<size_t>(block_m) * head_dim);
  std::vector<float> hk(static_cast<size_t>(seq_n) * head_dim);
  std::vector<float> hv(hk.size());
  makeInputs(a, hq, hk, hv);
  std::vector<_Float16> pq = packHalf(hq), pk = packHalf(hk), pv = packHalf(hv);
  std::memcpy(q, pq.data(), pq.size() * 2);
  std::memcpy(k, pk.data(), pk.size() * 2);
  std::memcpy(v, pv.data(), pv.size() * 2);
  std::vector<float> ref = computeReference(a, hq, hk, hv);
  std::memcpy(out, ref.data(), ref.size() * sizeof(float));
}
#endif

} // extern "C"
