// The thread's last error message, shared by the device ABI and the host
// mirror so rl_sampler_last_error() reports both.
#pragma once
#include <string>

namespace rl {
void set_last_error(const std::string &msg);
}
