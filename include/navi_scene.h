/*
 * navi_scene.h — C ABI of the host scene compiler (libnavi_scene.so).
 *
 * Produces .gmdag DAG words (docs/GMDAG.md:161-228 of the seismael/navi
 * checkout) from procedural scenes under the rules of the reference compiler's
 * build_recursive / compressToDAG (projects/voxel-dag/src/compiler.cpp:563-674).
 * The reference compiler takes meshes through Assimp (compiler.cpp:260-336);
 * these entry points take analytic primitives instead. Host memory only.
 *
 * prims: n_prims rows of 7 doubles (type, p0..p5):
 *   0 sphere         (cx, cy, cz, r, -, -)
 *   1 solid box      (lo x, lo y, lo z, hi x, hi y, hi z)
 *   2 room interior  (lo xyz, hi xyz): free inside, solid outside
 * Sample (x, y, z) sits at bmin + (x, y, z) * voxel and holds
 * min(|min_i sdf_i|, trunc).
 */
#ifndef NAVI_SCENE_H
#define NAVI_SCENE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dense [z][y][x] float32 samples (res^3 floats into `out`). 0 on success. */
int navi_scene_sample_dense(const double* prims, int32_t n_prims, const double* bmin, double voxel,
                            int32_t res, double trunc, float* out, int32_t threads);

/* DAG words of a dense [z][y][x] grid (replaces Compiler::compressToDAG,
 * compiler.cpp:661-674). *out_words is malloc'd (free with navi_scene_free).
 * quirk_half = 1 selects the reference's truncating float_to_half
 * (compiler.cpp:542-560); 0 rounds to nearest even. Returns the word count,
 * 0 on failure. */
uint64_t navi_dag_compile_dense(const float* grid, int32_t res, float voxel_size, int32_t quirk_half,
                                uint64_t** out_words);

/* DAG words of a procedural scene, identical to sampling densely and calling
 * navi_dag_compile_dense, without materialising the grid. voxel_size_f32 is
 * the header voxel the build rules use. Returns the word count, 0 on failure. */
uint64_t navi_scene_compile(const double* prims, int32_t n_prims, const double* bmin, double voxel,
                            int32_t res, double trunc, float voxel_size_f32, int32_t quirk_half,
                            int32_t threads, uint64_t** out_words, uint64_t* out_active_bricks);

void navi_scene_free(void* p);
const char* navi_scene_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NAVI_SCENE_H */
