// Dispatch of library steps (materializing ops that are not fusion groups).
#include "runtime.h"

namespace pjrtx {

void run_library_step(Device* dev, const Program& prog, const Step& step, std::vector<MemRef>& vals) {
  (void)dev;
  (void)prog;
  (void)vals;
  fail(Code::kUnimplemented, std::string("library op not available in this build: ") + lib_kind_name(step.lib));
}

}  // namespace pjrtx
