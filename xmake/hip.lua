-- MI355X (gfx950) build of libllaisys.so from llaisys_amd/csrc, for the reference's
-- xmake.lua (which includes its device targets the same way, xmake.lua:7-18):
--
--     option("amd-gpu")
--         set_default(false)
--         set_showmenu(true)
--         set_description("Build libllaisys.so for AMD MI355X (HIP, gfx950)")
--     option_end()
--     if has_config("amd-gpu") then
--         includes("xmake/hip.lua")
--     end
--
-- then `xmake f --amd-gpu=y && xmake build llaisys-hip && xmake install llaisys-hip`.
-- The target is the whole library (its own tensor, runtime, device and op layers), built
-- with the flags of llaisys_amd/csrc/Makefile, which stays the reference build of this
-- tree:
--   host C++ and HIP:  -O3 -std=c++17 -fPIC -Wall -ffp-contract=off (products and sums
--                      round as in the reference CPU kernels)
--   HIP only:          --offload-arch=gfx950, and no packed f32 VALU instructions
--                      (-Xclang -target-feature -Xclang -packed-fp32-ops)
-- The kernels need hipcc from ROCm (HIPCC, else /opt/rocm/bin/hipcc).

local hip_flags = {"-O3", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off",
                   "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"}

rule("llaisys-hip-gfx950")
    set_extensions(".hip")
    on_build_file(function (target, sourcefile, opt)
        import("core.project.depend")
        local objectfile = target:objectfile(sourcefile)
        table.insert(target:objectfiles(), objectfile)
        local hipcc = os.getenv("HIPCC") or "/opt/rocm/bin/hipcc"
        local args = {"-c"}
        for _, f in ipairs(target:values("llaisys.hip_flags")) do table.insert(args, f) end
        for _, dir in ipairs(target:get("includedirs")) do table.insert(args, "-I" .. dir) end
        table.insert(args, sourcefile)
        table.insert(args, "-o")
        table.insert(args, objectfile)
        depend.on_changed(function ()
            os.mkdir(path.directory(objectfile))
            os.vrunv(hipcc, args)
        end, {dependfile = target:dependfile(objectfile), files = {sourcefile}})
    end)
rule_end()

target("llaisys-hip")
    set_kind("shared")
    set_basename("llaisys")
    set_languages("cxx17")
    add_rules("llaisys-hip-gfx950")
    set_values("llaisys.hip_flags", hip_flags)
    add_includedirs(path.join(os.scriptdir(), "../include"))
    -- host C++ goes through hipcc too (it includes the HIP runtime headers)
    set_toolset("cxx", os.getenv("HIPCC") or "/opt/rocm/bin/hipcc")
    set_toolset("sh", os.getenv("HIPCC") or "/opt/rocm/bin/hipcc")
    add_cxflags("-O3", "-fPIC", "-Wall", "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__")
    add_shflags("--offload-arch=gfx950", "-Wl,--no-undefined")
    add_files(path.join(os.scriptdir(), "../llaisys_amd/csrc/utils/*.cpp"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/core/*.cpp"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/tensor/*.cpp"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/device/*.cpp"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/ops/*.cpp"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/capi/capi.cc"),
              path.join(os.scriptdir(), "../llaisys_amd/csrc/kernels/*.hip"))
    set_installdir(".")
    after_install(function (target)
        -- the reference loader looks for libllaisys.so next to its ctypes package
        os.cp(target:targetfile(), "python/llaisys/libllaisys/")
    end)
target_end()
