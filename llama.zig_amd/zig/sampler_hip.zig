//! sampler_hip.zig -- llama.zig's token sampler on an MI355X, as a drop-in for
//! src/sampler.zig.
//!
//! The public declarations have the reference's names, types and meaning
//! (sampler.zig:4-41):
//!     pub const SamplerConfig = struct { ... }                 sampler.zig:4-13
//!     pub const Sampler = struct {
//!         pub fn init(cfg: SamplerConfig) Sampler               sampler.zig:19-24
//!         pub fn sample(self: *Sampler, allocator, logits, prev_tokens) !TokenID
//!                                                               sampler.zig:26-28
//!     }
//!     pub fn sampleArgmax(logits: []const f32) TokenID          sampler.zig:31-41
//! so a caller switches by changing its import line only:
//!     const sampler = @import("sampler_hip.zig");   // main.zig:11, engine.zig:6
//! and main.zig:518,667 / engine.zig:215,355 stay as they are.
//!
//! The sampling chain (repetition penalty, softmax, top-k, top-p, min-p,
//! typical-p, the draw: sampler.zig:43-169) runs in libllzsample.so through
//! its C ABI (include/llz_sampler.h).  The PRNG stays here: `prng` is the
//! reference's own std.Random.DefaultPrng, seeded as sampler.zig:22 seeds
//! it, and the uniform of each row is drawn from it on the host.  The library
//! reports whether the row reached the draw (sampler.zig:162); when it did
//! not (temperature <= 0, sum <= 0, empty kept set) the draw is undone, so
//! the stream advances exactly as the reference's does.
//!
//! Differences a caller can see, all outside the reference's signatures:
//!   * the first `sample` of the process opens the GPU (device 0): `init`
//!     stays infallible, and every Sampler shares that one device handle
//!     (a stream and buffers sized to the longest row seen), each call
//!     passing its own configuration, so a Sampler created per request
//!     (engine.zig:215) costs nothing on the device and nothing leaks;
//!   * `sample` can fail with error.GpuUnavailable or error.GpuFailure as
//!     well as error.OutOfMemory (callers use `try`, as main.zig:667 does);
//!   * `deinit` exists for callers that want it and does nothing: the shared
//!     handle lives until the process ends;
//!   * `allocator` is accepted and unused: the library keeps its own device
//!     buffers;
//!   * calls from several threads are serialised on the shared handle.
const std = @import("std");
const tokenizer = @import("tokenizer.zig");

pub const SamplerConfig = struct {
    temperature: f32 = 0.8,
    top_k: u32 = 0,
    top_p: f32 = 0.9,
    min_p: f32 = 0.0,
    typical_p: f32 = 1.0,
    seed: u64 = 0,
    repetition_window: u32 = 32,
    repetition_penalty: f32 = 1.1,
};

/// The C ABI of libllzsample.so (include/llz_sampler.h).
pub const c = struct {
    /// llz_sampler_config: SamplerConfig's fields in its order, as an extern
    /// struct (the u32 before `seed` is the padding C inserts there too).
    pub const Config = extern struct {
        temperature: f32,
        top_k: u32,
        top_p: f32,
        min_p: f32,
        typical_p: f32,
        reserved: u32 = 0,
        seed: u64,
        repetition_window: u32,
        repetition_penalty: f32,
    };
    pub const Handle = opaque {};

    pub const OK: c_int = 0;
    pub const E_INVALID_ARG: c_int = -1;
    pub const E_WORKSPACE: c_int = -2;
    pub const E_HIP: c_int = -3;
    pub const E_OOM: c_int = -4;
    pub const E_NO_DEVICE: c_int = -5;

    pub extern "llzsample" fn llz_sampler_create(cfg: *const Config, device: i32, out: *?*Handle) c_int;
    pub extern "llzsample" fn llz_sampler_sample_config(
        s: *Handle,
        cfg: *const Config,
        logits: [*]const f32,
        n: i32,
        prev_tokens: ?[*]const u32,
        n_prev: i32,
        u: f32,
        token: *u32,
        consumed: *u8,
    ) c_int;
};

/// The process's device handle, shared by every Sampler (each call passes its
/// own configuration), opened by the first `sample`; calls are serialised.
var shared_gpu: ?*c.Handle = null;
var shared_lock: std.Thread.Mutex = .{};

fn sharedGpu() !*c.Handle {
    if (shared_gpu) |h| return h;
    const cfg = toC(.{});
    var h: ?*c.Handle = null;
    const rc = c.llz_sampler_create(&cfg, 0, &h);
    if (rc != c.OK) return mapError(rc);
    shared_gpu = h;
    return h.?;
}

fn toC(cfg: SamplerConfig) c.Config {
    return .{
        .temperature = cfg.temperature,
        .top_k = cfg.top_k,
        .top_p = cfg.top_p,
        .min_p = cfg.min_p,
        .typical_p = cfg.typical_p,
        .seed = cfg.seed,
        .repetition_window = cfg.repetition_window,
        .repetition_penalty = cfg.repetition_penalty,
    };
}

pub const Sampler = struct {
    cfg: SamplerConfig,
    prng: std.Random.DefaultPrng,

    pub fn init(cfg: SamplerConfig) Sampler {
        return .{
            .cfg = cfg,
            .prng = std.Random.DefaultPrng.init(if (cfg.seed != 0) cfg.seed else 0xDEADBEEF),
        };
    }

    pub fn sample(self: *Sampler, allocator: std.mem.Allocator, logits: []const f32, prev_tokens: []const tokenizer.TokenID) !tokenizer.TokenID {
        _ = allocator;
        if (logits.len == 0 or logits.len > std.math.maxInt(i32) or prev_tokens.len > std.math.maxInt(i32))
            return error.InvalidLength;
        shared_lock.lock();
        defer shared_lock.unlock();
        const gpu = try sharedGpu();
        // The draw sampler.zig:162 would make; undone below when the row
        // leaves the chain before it.
        const before = self.prng;
        const u = self.prng.random().float(f32);
        const cfg = toC(self.cfg);
        var token: u32 = 0;
        var consumed: u8 = 0;
        const rc = c.llz_sampler_sample_config(
            gpu,
            &cfg,
            logits.ptr,
            @intCast(logits.len),
            if (prev_tokens.len > 0) prev_tokens.ptr else null,
            @intCast(prev_tokens.len),
            u,
            &token,
            &consumed,
        );
        if (rc != c.OK or consumed == 0) self.prng = before;
        if (rc != c.OK) return mapError(rc);
        return token;
    }

    /// Nothing to release: the device handle is the process's shared one
    /// (see the file comment).  Kept for callers that pair init with deinit.
    pub fn deinit(self: *Sampler) void {
        _ = self;
    }
};

fn mapError(rc: c_int) error{ OutOfMemory, GpuUnavailable, GpuFailure, InvalidLength } {
    return switch (rc) {
        c.E_OOM => error.OutOfMemory,
        c.E_NO_DEVICE => error.GpuUnavailable,
        c.E_INVALID_ARG => error.InvalidLength,
        else => error.GpuFailure,
    };
}

/// The first index of the largest logit (ties keep the earliest), on the
/// host: the reference's greedy helper, used by callers directly.
pub fn sampleArgmax(logits: []const f32) tokenizer.TokenID {
    var best: usize = 0;
    var best_v: f32 = logits[0];
    var i: usize = 1;
    while (i < logits.len) : (i += 1) {
        if (logits[i] > best_v) {
            best_v = logits[i];
            best = i;
        }
    }
    return @intCast(best);
}

test "seeded samplers on the GPU repeat themselves" {
    const cfg = SamplerConfig{ .temperature = 1.0, .top_p = 1.0, .repetition_penalty = 1.0, .seed = 42 };
    var a = Sampler.init(cfg);
    defer a.deinit();
    var b = Sampler.init(cfg);
    defer b.deinit();
    const logits = [_]f32{ 1.0, 2.0, 0.5, 3.0 };
    for (0..16) |_| {
        const ta = try a.sample(std.testing.allocator, &logits, &.{});
        const tb = try b.sample(std.testing.allocator, &logits, &.{});
        try std.testing.expectEqual(ta, tb);
    }
}

test "top-k 1 on the GPU is the argmax" {
    var s = Sampler.init(.{ .temperature = 1.0, .top_k = 1, .top_p = 1.0, .repetition_penalty = 1.0, .seed = 7 });
    defer s.deinit();
    const logits = [_]f32{ 0.1, 4.0, -2.0, 3.9 };
    try std.testing.expectEqual(@as(tokenizer.TokenID, 1), try s.sample(std.testing.allocator, &logits, &.{}));
    try std.testing.expectEqual(sampleArgmax(&logits), try s.sample(std.testing.allocator, &logits, &.{}));
}

test "rows that exit before the draw leave the PRNG untouched" {
    var s = Sampler.init(.{ .temperature = 0.0, .seed = 3 });
    defer s.deinit();
    const before = s.prng;
    const logits = [_]f32{ 0.0, 5.0, 5.0 };
    try std.testing.expectEqual(@as(tokenizer.TokenID, 1), try s.sample(std.testing.allocator, &logits, &.{}));
    try std.testing.expectEqual(before.s, s.prng.s);
}
