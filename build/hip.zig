//! The HIP half of the root build for the DiT joint-attention path on MI355X (gfx950), in place of build/cuda.zig for
//! that path: hipcc compiles the kernels of kernels/hip (this repository's localrouter_amd/csrc) into liblr_attn.so,
//! the plain C ABI of include/lr_attn.h, lr_rope.h and lr_mmdit.h, and the module `lr_attn`
//! (src/engines/hip/lr_attn.zig) holds its extern declarations and the engines' call-site helpers.
//! `-Dhipcc=<hipcc>` builds the library; without it the `lr-attn` step fails and the module is host-only.
//!
//! Where build/cuda.zig compiles fatbins with nvcc and embeds them for launch by symbol (build/cuda.zig:39-96), the
//! HIP path links a shared library and binds it by name: no images, no symbol tables, no per-call launch packs.

const std = @import("std");

/// One translation unit of the library and the hipcc flags it needs beyond `hip_flags`.
const Source = struct { file: []const u8, extra: []const []const u8 = &.{} };

/// The device sources (each a HIP translation unit for gfx950). attn_stream.hip needs its 32-slot step fully
/// unrolled, so that no register array is indexed at run time (which would put it in scratch).
const sources = [_]Source{
    .{ .file = "attn_fwd.hip" },
    .{ .file = "attn_stream.hip", .extra = &.{ "-mllvm", "-pragma-unroll-threshold=1000000" } },
    .{ .file = "kv_image.hip" },
    .{ .file = "rms_rope.hip" },
    .{ .file = "int8_attn.hip" },
    .{ .file = "keys.hip" },
    .{ .file = "lr_abi.hip" },
    .{ .file = "mmdit.hip" },
};

/// hipcc flags of every device source: gfx950 only, no packed-fp32 instruction selection (v_pk_*_f32 are left to
/// nothing), C++17, position-independent code for the shared library.
const hip_flags = [_][]const u8{
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
};

pub const LrAttn = struct {
    /// The extern declarations (src/engines/hip/lr_attn.zig), linked against liblr_attn.so when it is built.
    module: *std.Build.Module,
    /// liblr_attn.so (null without -Dhipcc); installed as lib/liblr_attn.so by the `lr-attn` step.
    lib: ?std.Build.LazyPath,
    /// The `lr-attn` step: build and install the library.
    step: *std.Build.Step,
    /// Host tests of the bindings module (constants, error mapping); no GPU and no library needed.
    tests: *std.Build.Step,
};

/// Adds `-Dhipcc`, `-Drocm` and the `lr-attn` / `test-lr-attn` steps; returns the module `lr_attn`.
pub fn lrAttn(b: *std.Build, target: std.Build.ResolvedTarget, optimize: std.builtin.OptimizeMode) LrAttn {
    const hipcc = b.option([]const u8, "hipcc", "hipcc that builds liblr_attn.so for gfx950 (e.g. /opt/rocm/bin/hipcc)");
    const rocm = b.option([]const u8, "rocm", "ROCm prefix: hipBLASLt and amdhip64 for the link") orelse "/opt/rocm";
    const step = b.step("lr-attn", "Build and install liblr_attn.so (needs -Dhipcc)");

    var lib: ?std.Build.LazyPath = null;
    if (hipcc) |cc| {
        // the compiler's version text is an input of every object, so a new ROCm rebuilds them all
        const version_run = b.addSystemCommand(&.{ cc, "--version" });
        version_run.has_side_effects = true;
        const version = version_run.captureStdOut(.{});

        const link = b.addSystemCommand(&.{ cc, "--offload-arch=gfx950", "-shared", "-fPIC" });
        for (sources) |src| {
            const run = b.addSystemCommand(&.{cc});
            run.addFileInput(version);
            run.addArgs(&hip_flags);
            run.addArgs(src.extra);
            // lr_abi.hip and mmdit.hip include ../../include/lr_*.h: kernels/hip sits two levels below the root
            run.addArgs(&.{ "-MD", "-MF" });
            _ = run.addDepFileOutputArg2(b.fmt("{s}.d", .{src.file}), .{});
            run.addArg("-c");
            run.addFileArg(b.path(b.fmt("kernels/hip/{s}", .{src.file})));
            run.addArg("-o");
            link.addFileArg(run.addOutputFileArg(b.fmt("{s}.o", .{std.fs.path.stem(src.file)})));
        }
        // the host RoPE table builders (include/lr_rope.h): plain C++, no FMA contraction, so that the tables are
        // the same bits as the engines' own builders
        const rope = b.addSystemCommand(&.{ "c++", "-O2", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off", "-c" });
        rope.addFileArg(b.path("kernels/hip/rope_host.cpp"));
        rope.addArg("-o");
        link.addFileArg(rope.addOutputFileArg("rope_host.o"));
        // the MMDiT block's projections and MLP run on hipBLASLt
        link.addArgs(&.{ b.fmt("-L{s}/lib", .{rocm}), "-lhipblaslt", "-o" });
        lib = link.addOutputFileArg("liblr_attn.so");
        step.dependOn(&b.addInstallFile(lib.?, "lib/liblr_attn.so").step);
    } else step.dependOn(&b.addFail("the lr-attn step needs -Dhipcc=<hipcc>").step);

    const m = b.createModule(.{
        .root_source_file = b.path("src/engines/hip/lr_attn.zig"),
        .target = target,
        .optimize = optimize,
    });
    if (lib) |so| {
        m.addLibraryPath(so.dirname());
        m.linkSystemLibrary("lr_attn", .{});
        m.addLibraryPath(.{ .cwd_relative = b.fmt("{s}/lib", .{rocm}) });
        m.linkSystemLibrary("amdhip64", .{});
    }

    // host tests: the same file without the library (the tests reference no extern function)
    const host = b.createModule(.{
        .root_source_file = b.path("src/engines/hip/lr_attn.zig"),
        .target = target,
        .optimize = optimize,
    });
    const tests = b.step("test-lr-attn", "Host tests of the liblr_attn.so bindings");
    tests.dependOn(&b.addRunArtifact(b.addTest(.{ .root_module = host })).step);
    return .{ .module = m, .lib = lib, .step = step, .tests = tests };
}
