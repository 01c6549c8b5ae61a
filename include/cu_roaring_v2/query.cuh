// Drop-in name of the reference header; see query.hpp.
#pragma once
#include "cu_roaring_v2/query.hpp"
