// The view type lives in resources.hpp (reference: include/raft/core/device_mdspan.hpp:1-3).
#pragma once

#include <raft/core/resources.hpp>
