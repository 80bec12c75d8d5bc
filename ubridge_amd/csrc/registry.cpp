// registry.cpp -- kernel-by-name lookup and launch, the counterpart of the
// reference's DeviceExecutor function_map (src/device_executor.rs:110-531)
// and GcuLaunchAsync::launch (src/gcu_launch.rs:121-181,259-328).
//
// A caller that launched "dequantize_block_q8_0_bf16" from module "quant" by
// name with an array of pointers to its positional arguments keeps doing so:
// ubridge_get_function(name, module) returns a handle (NULL if unknown, where
// the reference silently returned a no-op function), and ubridge_launch(handle,
// args, stream) unpacks the arguments with the reference's signature and calls
// the entry point, which picks its own grid for MI355X (the reference's
// GcuLaunchConfig <<<2, 12>>> tiling hints do not apply to 256 CUs).
#include <string.h>

#include "common.h"
#include "registry.h"

namespace {

struct Entry {
  const char* module;
  const char* name;
  ub_thunk fn;
};

const Entry* table(size_t* n);

}  // namespace

UB_API const void* ubridge_get_function(const char* name, const char* module) {
  if (!name) return nullptr;
  size_t n;
  const Entry* t = table(&n);
  for (size_t i = 0; i < n; i++)
    if (!strcmp(t[i].name, name) && (!module || !strcmp(t[i].module, module))) return &t[i];
  ub_set_error(UB_ERR_INVALID_ARG, "ubridge_get_function: no kernel '%s' in module '%s'", name,
               module ? module : "*");
  return nullptr;
}

UB_API int ubridge_has_function(const char* name) {
  size_t n;
  const Entry* t = table(&n);
  for (size_t i = 0; i < n; i++)
    if (name && !strcmp(t[i].name, name)) return 1;
  return 0;
}

UB_API int ubridge_num_functions(void) {
  size_t n;
  table(&n);
  return (int)n;
}

UB_API const char* ubridge_function_name(int i) {
  size_t n;
  const Entry* t = table(&n);
  return (i >= 0 && (size_t)i < n) ? t[i].name : nullptr;
}

UB_API int ubridge_launch(const void* handle, void** args, void* stream) {
  if (!handle) return ub_set_error(UB_ERR_INVALID_ARG, "ubridge_launch: null function handle");
  if (!args) return ub_set_error(UB_ERR_INVALID_ARG, "ubridge_launch: null argument array");
  const Entry* e = (const Entry*)handle;
  ubridge_last_error();  // clear any stale error so the thunk's result is its own
  e->fn(args, stream);
  int rc = ubridge_last_error();
  if (rc) ub_set_error(rc, "%s", ubridge_last_error_string());
  return rc;
}

namespace {
#define UB_REG(mod, nm) {mod, #nm, ub_thunk_##nm},
const Entry kTable[] = {
    UB_REGISTRY_ENTRIES(UB_REG)
};
#undef UB_REG
const Entry* table(size_t* n) {
  *n = sizeof(kTable) / sizeof(kTable[0]);
  return kTable;
}
}  // namespace
