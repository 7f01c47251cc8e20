// ref_matmul_shim.cpp -- builds the reference runner's CPU-side code, from the
// reference checkout, into oracle/_ref/libref_matmul.so.
//
// TEST INFRASTRUCTURE ONLY (never shipped, never loaded by the product).  It
// uses the reference's own trick (test/Integration/Inputs/
// wave_matmul_rand_int_test.cpp:9-10): define WAVE_MATMUL_CALIBRATE_RUNNER_NO_MAIN
// and include the runner source where it lies (path given by -include on the
// compile line in oracle/Makefile), then export C entry points over the
// runner's own functions so tests/golden/make_golden.py can record vectors.
#include <cstdint>
#include <cstring>

extern "C" {

void ref_make_input_bytes(int rows, int k, int type, int seed, int stream,
                          int all_ones, int rand_int, int hpl, uint8_t *out) {
  std::vector<uint8_t> b =
      makeInputBytes(rows, k, type == 2 ? InputType::BF16 : InputType::F16,
                     seed, stream, all_ones != 0, rand_int != 0, hpl != 0);
  std::memcpy(out, b.data(), b.size());
}

float ref_half_to_float(uint16_t h) { return halfToFloat(h); }
uint16_t ref_float_to_half_bits(float v) { return floatToHalfBits(v); }
uint16_t ref_float_to_bf16_bits(float v) { return floatToBF16Bits(v); }
float ref_random_input_value(uint32_t *state) { return randomInputValue(*state); }
uint32_t ref_rand_state(int seed, int stream) { return randState(seed, stream); }
float ref_hipblaslt_rand_int(size_t i) { return hipblasLtRandInt(i); }
float ref_hipblaslt_hpl(size_t i) { return hipblasLtHpl(i); }

// C[m][n] via computeExpectedElement (float accumulate) for the given mode,
// then roundExpectedOutput for the requested output type (0 f32, 1 f16, 2 bf16).
void ref_gemm_expected(int m, int n, int k, int type, int seed, int mode,
                       int out_type, double *out) {
  Args a;
  a.m = m;
  a.n = n;
  a.k = k;
  a.inputType = type == 2 ? InputType::BF16 : InputType::F16;
  a.seed = seed;
  a.allOnes = mode == 1;
  a.randInt = mode == 2;
  a.hpl = mode == 3;
  a.cType = out_type == 1 ? CType::F16 : out_type == 2 ? CType::BF16 : CType::F32;
  HostInputs in = makeHostInputs(a);
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j)
      out[static_cast<size_t>(i) * n + j] =
          roundExpectedOutput(computeExpectedElement(in, a, i, j), a.cType);
}

// getOutputCoordinate for a 16x16 single-wave tile (rand_int_test.cpp:112-141).
void ref_output_coordinate(int wave_size, int wmma, int index, int *m, int *n) {
  Args a;
  a.m = 16;
  a.n = 16;
  a.bm = 1;
  a.bn = 1;
  a.waveMTiles = 1;
  a.waveNTiles = 1;
  a.waveSize = wave_size;
  a.accumulatorLayout = wmma ? AccumulatorLayout::Wmma : AccumulatorLayout::Mfma;
  OutputCoordinate c = getOutputCoordinate(a, index);
  *m = c.m;
  *n = c.n;
}

// getOutputCoordinate of a tile-packed C (runner.cpp:772-834) for the
// reference blocking (bm, bn, wave_m_tiles, wave_n_tiles) of an m x n output,
// gfx950 MFMA accumulators (wave64).
void ref_tile_packed_coordinate(int m, int n, int bm, int bn, int wmt, int wnt,
                                int index, int *om, int *on) {
  Args a;
  a.m = m;
  a.n = n;
  a.bm = bm;
  a.bn = bn;
  a.waveMTiles = wmt;
  a.waveNTiles = wnt;
  a.waveSize = 64;
  a.accumulatorLayout = AccumulatorLayout::Mfma;
  OutputCoordinate c = getOutputCoordinate(a, index);
  *om = c.m;
  *on = c.n;
}

// getStreamKWorkspaceSizes + makeLaunchShape for the Stream-K ABI.
void ref_streamk_workspace(int m, int n, int k, int workers, uint64_t *scratch,
                           uint64_t *counters, int *grid_x, int *block) {
  Args a;
  a.m = m;
  a.n = n;
  a.k = k;
  a.bm = 2;
  a.bn = 2;
  a.waveMTiles = 8;
  a.waveNTiles = 8;
  a.waveKTiles = 2;
  a.waveSize = 64;
  a.cType = CType::F16;
  a.kernelABI = KernelABI::StreamK;
  a.streamKWorkers = workers;
  StreamKWorkspaceSizes s = getStreamKWorkspaceSizes(a);
  *scratch = s.scratchBytes;
  *counters = s.counterElements;
  LaunchShape l = makeLaunchShape(a);
  *grid_x = l.gridX;
  *block = l.blockThreads;
}

// MXFP4 generators (runner.cpp:1135-1150, :1208-1220): packed e2m1 codes and
// group-major e8m0 scales for `rows` x `k`.
void ref_mxfp4_input_bytes(int rows, int k, int seed, int stream, int all_ones,
                           uint8_t *out) {
  std::vector<uint8_t> b = makeMXFP4InputBytes(
      static_cast<size_t>(rows) * k, seed, stream, all_ones != 0);
  std::memcpy(out, b.data(), b.size());
}
void ref_mxfp4_scale_bytes(int rows, int k, int seed, int stream, int all_ones,
                           uint8_t *out) {
  std::vector<uint8_t> b = makeMXFP4ScaleBytes(rows, k, seed, stream, all_ones != 0);
  std::memcpy(out, b.data(), b.size());
}
float ref_mxfp4_code_to_float(int code) { return mxfp4CodeToFloat(static_cast<uint8_t>(code)); }
float ref_e8m0_to_float(int raw) { return e8m0ToFloat(static_cast<uint8_t>(raw)); }

// The runner's MXFP4 expected output: makeHostInputs + computeExpectedElement
// + roundExpectedOutput (runner.cpp:1436-1456, :1565-1597).
void ref_gemm_mxfp4_expected(int m, int n, int k, int seed, int all_ones,
                             int out_type, double *out) {
  Args a;
  a.m = m;
  a.n = n;
  a.k = k;
  a.inputType = InputType::MXFP4;
  a.waveSize = 64;
  a.seed = seed;
  a.allOnes = all_ones != 0;
  a.cType = out_type == 1 ? CType::F16 : out_type == 2 ? CType::BF16 : CType::F32;
  HostInputs in = makeHostInputs(a);
  for (int i = 0; i < m; ++i)
    for (int j = 0; j < n; ++j)
      out[static_cast<size_t>(i) * n + j] =
          roundExpectedOutput(computeExpectedElement(in, a, i, j), a.cType);
}

// AITER layouts (runner.cpp:1223-1283): shuffled B bytes and scale bytes.
void ref_mxfp4_aiter_b(const uint8_t *in, int n, int k, uint8_t *out) {
  Args a;
  a.n = n;
  a.k = k;
  std::vector<uint8_t> c(in, in + static_cast<size_t>(n) * (k / 2));
  std::vector<uint8_t> s = makeAITERBBytes(c, a);
  std::memcpy(out, s.data(), s.size());
}
size_t ref_mxfp4_aiter_scales(const uint8_t *in, int rows, int k, uint8_t *out) {
  Args a;
  a.k = k;
  std::vector<uint8_t> c(in, in + static_cast<size_t>(rows) * (k / 32));
  std::vector<uint8_t> s = makeAITERScaleBytes(c, rows, a);
  if (out)
    std::memcpy(out, s.data(), s.size());
  return s.size();
}

} // extern "C"
