-- xmake entry for llaisys_amd (the reference's build hooks: xmake.lua:10-19,
-- xmake/cpu.lua). The library's device runtime and kernels are HIP for
-- AMD Instinct MI355X (gfx950); `xmake f --amd-gpu=y && xmake` builds
-- llaisys_amd/libllaisys/libllaisys.so from the same sources and flags as
-- llaisys_amd/build.py.
add_rules("mode.debug", "mode.release")
set_encodings("utf-8")

add_includedirs("include")

-- AMD --
option("amd-gpu")
    set_default(true)
    set_showmenu(true)
    set_description("Compile the HIP implementations for AMD Instinct MI355X (gfx950)")
option_end()

if has_config("amd-gpu") then
    add_defines("ENABLE_AMD_API")
    includes("xmake/hip.lua")
else
    -- Every part of this library (host ops included) links the HIP runtime.
    target("llaisys")
        set_kind("phony")
        on_build(function (target)
            raise("llaisys_amd needs the amd-gpu option (xmake f --amd-gpu=y)")
        end)
    target_end()
end
