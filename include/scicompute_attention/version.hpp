#pragma once

#include "scicompute_attention/export.hpp"

#define SCI_ATTENTION_VERSION_MAJOR 0
#define SCI_ATTENTION_VERSION_MINOR 1
#define SCI_ATTENTION_VERSION_PATCH 0
#define SCI_ATTENTION_VERSION_STRING "0.1.0"

namespace sca {

// "major.minor.patch" of the API this library implements.
SCI_ATTENTION_API const char* VersionString() noexcept;

// Identifies this implementation ("mi355x-hip-gfx950").
SCI_ATTENTION_API const char* BuildFlavor() noexcept;

}  // namespace sca
