/*
 * pjrt_amd.h -- the one symbol of the PJRT plugin library (libpjrt_amd.so).
 *
 * jaxlib loads a PJRT plugin by path and calls exactly this function (lowercase
 * "rt"); it replaces the reference plugin's export of the same name
 * (/root/reference/pjrt_plugin/src/plugin.cc:1083-1087, table built at 994-1081).
 *
 * The returned table is PJRT C API 0.112 (the layout of openxla's
 * xla/pjrt/c/pjrt_c_api.h at that version, restated for the calls this plugin
 * implements in pjrt-ocl_amd/csrc/pjrt_abi.h).  Platform name "mi355x"; one
 * device; compile runs the Python lowering service
 * (pjrt_amd/lower_service.py), execute runs the megakernel VM of libvmrt.so.
 * Slots the plugin does not provide return PJRT_Error_Code_UNIMPLEMENTED with
 * the slot's name.
 */
#ifndef PJRT_AMD_H_
#define PJRT_AMD_H_

#ifdef __cplusplus
extern "C" {
#endif

struct PJRT_Api;

const struct PJRT_Api* GetPjrtApi(void);

#ifdef __cplusplus
}
#endif

#endif /* PJRT_AMD_H_ */
