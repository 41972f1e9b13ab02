-- HIP target for gfx950: every .cpp and .hip under llaisys_amd/csrc is
-- compiled by hipcc as HIP and linked into one shared library, the file the
-- ctypes layer loads (llaisys_amd/libllaisys/libllaisys.so). The compile
-- flags below are the ones llaisys_amd/build.py passes; a test keeps the two
-- lists equal.
local rocm = os.getenv("ROCM_PATH") or "/opt/rocm"
local hipcc = os.getenv("HIPCC") or path.join(rocm, "bin", "hipcc")

-- HIP_FLAGS_BEGIN
local hip_flags = {
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fvisibility=hidden",
}
-- HIP_FLAGS_END

-- Per-source extra flags (llaisys_amd/build.py's EXTRA), keyed by the path
-- under llaisys_amd/csrc.
-- HIP_EXTRA_BEGIN
local hip_extra = {
    ["kernels/gemm.hip"] = {"-mllvm", "-amdgpu-mfma-vgpr-form"},
}
-- HIP_EXTRA_END

-- Compile one source with hipcc as HIP; the argument vector is passed as is
-- (paired -Xclang options must not be merged or de-duplicated).
rule("hip-gfx950")
    set_extensions(".hip", ".cpp")
    on_build_file(function (target, sourcefile, opt)
        local objectfile = target:objectfile(sourcefile)
        table.insert(target:objectfiles(), objectfile)
        os.mkdir(path.directory(objectfile))
        local argv = {"-x", "hip"}
        for _, f in ipairs(hip_flags) do table.insert(argv, f) end
        local rel = path.relative(sourcefile, path.join(os.projectdir(), "llaisys_amd", "csrc")):gsub("\\", "/")
        for _, f in ipairs(hip_extra[rel] or {}) do table.insert(argv, f) end
        table.insert(argv, "-I" .. path.join(os.projectdir(), "include"))
        table.insert(argv, "-c")
        table.insert(argv, sourcefile)
        table.insert(argv, "-o")
        table.insert(argv, objectfile)
        os.vrunv(hipcc, argv)
    end)
rule_end()

target("llaisys")
    set_kind("shared")
    add_rules("hip-gfx950")
    add_files("../llaisys_amd/csrc/**.cpp", "../llaisys_amd/csrc/**.hip")
    set_toolset("sh", hipcc)
    add_shflags("--offload-arch=gfx950", {force = true})
    after_build(function (target)
        -- the ctypes loader reads the library from the package directory
        -- (as python/llaisys/libllaisys/__init__.py:17-40 does)
        os.cp(target:targetfile(), path.join(os.projectdir(), "llaisys_amd", "libllaisys", "libllaisys.so"))
    end)
target_end()
