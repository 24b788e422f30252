// random.hpp -- the engine's host random generator (the reference's
// include/engine/random.hpp): Tensor::rand / randn draw the initial parameters
// from it, callers draw their own shuffles and synthetic data from it, and
// manual_seed() reseeds it. One generator shared by the process, with no
// synchronisation.
#ifndef ENGINE_RANDOM_HPP
#define ENGINE_RANDOM_HPP

#include <random>

namespace engine {

std::mt19937& global_rng();

}  // namespace engine

#endif  // ENGINE_RANDOM_HPP
