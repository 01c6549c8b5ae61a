// Drop-in name of the reference header; see to_csr.hpp.
#pragma once
#include "cu_roaring/detail/to_csr.hpp"
