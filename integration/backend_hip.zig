//! backend_hip.zig -- the quantized-matvec slots of `backend.Exec` on an
//! MI355X (gfx950), through libqwen35_hip.so (include/qwen35_hip.h).
//!
//! Drops in beside src/backend_cpu.zig: add `hip` to `backend.Kind` and
//! `.hip => @import("backend_hip.zig").HipBackend` to `selectBackend`
//! (src/backend.zig:741-748); `main.zig` then accepts `--backend hip`.  Build:
//! link `libqwen35_hip.so` (and `libamdhip64.so`) with `exe.linkSystemLibrary`
//! and `exe.addLibraryPath`, as `-Dcuda` does for the CUDA objects
//! (build.zig:212-245).
//!
//! What runs where.  This library implements the quantized matvec path
//! (`matvec`, `matvecPair`, `matvecBatchK`, `dequantRow`) on the GPU; every
//! other slot (norms, attention, recurrence, sampling) keeps the CPU backend's
//! implementation, which this backend embeds -- the same first slice the CUDA
//! backend started from (src/backend.zig:735-740).  So that both sides can
//! touch every activation, `allocBuf` regions are pinned host memory mapped
//! into the GPU's address space (hipHostMalloc, coherent): the CPU slots read
//! and write them as ordinary memory, the HIP kernels read x and write out
//! through the mapping, and each matvec slot waits for its launch before
//! returning, because the next CPU slot reads its output.
//!
//! Weights.  `loadLinear` takes the CPU backend's zero-copy view of the GGUF
//! tensor and uploads a packed quantized weight once
//! (qhip_backend_load_linear: consecutive loads are byte-adjacent on the
//! device, so an adjacent `matvecPair` is one launch).  The device copy is
//! found again by the view's host pointer, as CudaBackend.findDev does
//! (src/backend_cuda.zig:1738-1752).  `.f32` weights stay on the CPU path.
//!
//! Errors follow src/backend_cuda.zig:3836-3841: a failed launch prints the
//! library's message and zero-fills the output; nothing falls back to the CPU
//! silently.  `QWEN35_HIP_MAX_DEV_MIB` caps the device memory the backend
//! places (qhip_backend_set_mem_budget), as `QWEN35_CUDA_MAX_DEV_MIB` does
//! (src/backend_cuda.zig:1754-1760).
//!
//! Introspection and profiling.  `describe` is the library's one-line account
//! of the device, the bytes placed and the switches in use.  Under
//! `$QWEN35_PROF` the library times every matvec slot on the device (HIP event
//! pairs, read back lazily) and `reportProfile` / `profReport` print its
//! per-(slot, type, shape) table -- calls, device time, GB/s, the fraction of
//! HBM peak -- followed by the CPU backend's own table for the slots still on
//! the CPU, as the CUDA backend prints its per-type device table
//! (src/backend_cuda.zig:6647).  `$QWEN35_HIP_MVCHECK` cross-checks the first
//! matvec and the first batch of each weight type against the embedded CPU
//! backend and prints the comparison (src/backend_cuda.zig:4018-4114);
//! `$QWEN35_HIP_MVCHECK_ONLY=<type>` restricts it to one type.
const std = @import("std");
const backend = @import("backend.zig");
const gguf = @import("gguf.zig");
const CpuBackend = @import("backend_cpu.zig").CpuBackend;

// ---- include/qwen35_hip.h ----------------------------------------------------------

const QhipBackend = opaque {};
const QhipLinear = extern struct {
    dev: ?*const anyopaque,
    ttype: c_int,
    rows: c_int,
    cols: c_int,
    row_bytes: c_long,
};
const QHIP_DECLINE: c_int = -1;

extern fn qhip_error_string(err: c_int) [*:0]const u8;
extern fn qhip_backend_create(device: c_int, err: ?*c_int) ?*QhipBackend;
extern fn qhip_backend_destroy(be: ?*QhipBackend) void;
extern fn qhip_backend_name(be: ?*const QhipBackend) [*:0]const u8;
extern fn qhip_backend_load_linear(be: ?*QhipBackend, ttype: c_int, rows: c_int, cols: c_int,
    host_data: ?*const anyopaque, out: *QhipLinear) c_int;
extern fn qhip_backend_free_linear(be: ?*QhipBackend, w: *QhipLinear) void;
extern fn qhip_backend_prepare_linear(be: ?*QhipBackend, w: *const QhipLinear) c_int;
extern fn qhip_backend_alloc_scratch_k(be: ?*QhipBackend, max_cols: c_int, k: c_int) c_int;
extern fn qhip_backend_free_scratch(be: ?*QhipBackend) void;
extern fn qhip_backend_matvec(be: ?*QhipBackend, d_out: ?[*]f32, w: *const QhipLinear, d_x: ?[*]const f32) c_int;
extern fn qhip_backend_matvec_pair(be: ?*QhipBackend, d_out: ?[*]f32, a: *const QhipLinear, b: *const QhipLinear,
    d_x: ?[*]const f32) c_int;
extern fn qhip_backend_matvec_batch_k(be: ?*QhipBackend, d_out: ?[*]f32, w: *const QhipLinear,
    d_xK: ?[*]const f32, k: c_int) c_int;
extern fn qhip_backend_dequant_row(be: ?*QhipBackend, d_dst: ?[*]f32, w: *const QhipLinear, row: c_int) c_int;
extern fn qhip_backend_sync(be: ?*QhipBackend) c_int;
extern fn qhip_backend_set_mem_budget(be: ?*QhipBackend, bytes: usize) c_int;
extern fn qhip_backend_step_begin(be: ?*QhipBackend, pos: c_uint) void;
extern fn qhip_backend_step_end(be: ?*QhipBackend) void;
extern fn qhip_backend_describe(be: ?*QhipBackend) [*:0]const u8;
extern fn qhip_backend_set_profiling(be: ?*QhipBackend, on: c_int) c_int;
extern fn qhip_backend_prof_report(be: ?*QhipBackend, buf: ?[*]u8, len: c_long) c_long;

// ---- the HIP runtime (libamdhip64): pinned, device-mapped host memory ----------------
extern fn hipHostMalloc(ptr: *?*anyopaque, size: usize, flags: c_uint) c_int;
extern fn hipHostFree(ptr: ?*anyopaque) c_int;
const hipHostMallocMapped: c_uint = 0x2;
const hipHostMallocCoherent: c_uint = 0x40000000;

pub const HipBackend = struct {
    alloc: std.mem.Allocator,
    cpu: CpuBackend,
    be: ?*QhipBackend,
    /// device copies of uploaded weights, found by the host view's pointer
    resident: std.ArrayListUnmanaged(Resident) = .empty,
    /// pinned Buf regions, released by freeScratch
    pinned: std.ArrayListUnmanaged(*anyopaque) = .empty,
    /// `$QWEN35_HIP_MVCHECK`: on, the type it is restricted to, and the weight
    /// types already checked (one check per type and slot kind)
    mvcheck_on: bool = false,
    mvcheck_only: ?[]const u8 = null,
    mvcheck_seen: [64]bool = @splat(false),
    mvcheck_seen_k: [64]bool = @splat(false),

    const Resident = struct { host: [*]const u8, lin: QhipLinear };

    pub fn init(alloc: std.mem.Allocator, g: *const gguf.File) HipBackend {
        var err: c_int = 0;
        const be = qhip_backend_create(0, &err);
        if (be == null) std.debug.print("hip backend: device 0 unavailable: {s}\n", .{qhip_error_string(err)});
        if (be) |b| {
            if (std.posix.getenv("QWEN35_HIP_MAX_DEV_MIB")) |v| {
                const mib = std.fmt.parseInt(usize, std.mem.trim(u8, v, " "), 10) catch 0;
                if (mib != 0) _ = qhip_backend_set_mem_budget(b, mib << 20);
            }
            if (std.posix.getenv("QWEN35_PROF") != null) _ = qhip_backend_set_profiling(b, 1);
        }
        return .{
            .alloc = alloc,
            .cpu = CpuBackend.init(alloc, g),
            .be = be,
            .mvcheck_on = std.posix.getenv("QWEN35_HIP_MVCHECK") != null,
            .mvcheck_only = std.posix.getenv("QWEN35_HIP_MVCHECK_ONLY"),
        };
    }

    pub fn exec(self: *HipBackend) backend.Exec {
        return .{ .ptr = &self.cpu, .vtable = &vtable };
    }

    pub fn deinit(self: *HipBackend) void {
        for (self.resident.items) |*r| qhip_backend_free_linear(self.be, &r.lin);
        self.resident.deinit(self.alloc);
        freePinned(self);
        self.pinned.deinit(self.alloc);
        qhip_backend_destroy(self.be);
        self.be = null;
        self.cpu.deinit();
    }

    /// The context of every slot is the embedded CPU backend.
    fn self_(ctx: *anyopaque) *HipBackend {
        const cpu: *CpuBackend = @ptrCast(@alignCast(ctx));
        return @fieldParentPtr("cpu", cpu);
    }

    fn findDev(self: *HipBackend, host: [*]const u8) ?*const QhipLinear {
        for (self.resident.items) |*r| if (r.host == host) return &r.lin;
        return null;
    }

    fn freePinned(self: *HipBackend) void {
        for (self.pinned.items) |p| _ = hipHostFree(p);
        self.pinned.clearRetainingCapacity();
    }

    /// src/backend_cuda.zig:3836-3841: report, zero the output, never a CPU retreat.
    fn failed(what: []const u8, rc: c_int, out: backend.Buf) void {
        std.debug.print("hip backend: {s}: {s}\n", .{ what, qhip_error_string(rc) });
        @memset(out.slice(), 0);
    }

    /// Wait for the launch: the next slot may be a CPU slot reading `out`.
    fn finish(self: *HipBackend, what: []const u8, rc: c_int, out: backend.Buf) void {
        if (rc != 0) return failed(what, rc, out);
        const rs = qhip_backend_sync(self.be);
        if (rs != 0) failed(what, rs, out);
    }

    /// `$QWEN35_HIP_MVCHECK`: a debug cross-check, not a computation path
    /// (src/backend_cuda.zig:4018-4114).  The first matvec and the first
    /// batch of each weight type run once more on the embedded CPU backend
    /// into a temporary, and the two results are compared: relative L2 over
    /// the output (the parity bar, 1e-5) and the count of elements more than
    /// 2e-2 apart relative to max(|cpu|, 1e-3), the reference's per-element
    /// test.  `out` is only read; it and `x` are host-mapped Buf regions, and
    /// `finish` has waited for the launch.
    fn mvCheck(self: *HipBackend, out: backend.Buf, w: backend.LinearW, x: backend.Buf, k: usize) void {
        if (!self.mvcheck_on) return;
        const q = switch (w) {
            .quant => |q| q,
            .f32 => return,
        };
        if (self.mvcheck_only) |only| if (!std.mem.eql(u8, only, @tagName(q.ttype))) return;
        const ti: usize = @intCast(@intFromEnum(q.ttype));
        const seen = if (k == 1) &self.mvcheck_seen else &self.mvcheck_seen_k;
        if (ti >= seen.len or seen[ti]) return;
        seen[ti] = true;
        const n = q.rows * k;
        const ref = self.alloc.alloc(f32, n) catch return;
        defer self.alloc.free(ref);
        const rbuf = backend.Buf.wrap(ref);
        if (k == 1) CpuBackend.vtable.matvec(&self.cpu, rbuf, w, x) else CpuBackend.vtable.matvecBatchK(&self.cpu, rbuf, w, x, k);
        var num: f64 = 0;
        var den: f64 = 0;
        var bad: usize = 0;
        for (out.slice()[0..n], ref) |dv, cv| {
            const d = @as(f64, dv) - @as(f64, cv);
            num += d * d;
            den += @as(f64, cv) * @as(f64, cv);
            if (@abs(dv - cv) / @max(@abs(cv), 1e-3) > 2e-2) {
                if (bad < 3) std.debug.print("  MVCHECK row: dev={d} cpu={d}\n", .{ dv, cv });
                bad += 1;
            }
        }
        const rel = if (den > 0) @sqrt(num / den) else @sqrt(num);
        std.debug.print("MVCHECK[{s}] rows={d} cols={d} k={d} rel_l2={e} mismatched={d} {s}\n", .{
            @tagName(q.ttype), q.rows, q.cols(), k, rel, bad, if (rel <= 1e-5 and bad == 0) "ok" else "FAIL",
        });
    }

    // ---- slots on the GPU ---------------------------------------------------------------

    fn vLoadLinear(ctx: *anyopaque, name: []const u8) backend.LoadError!backend.LinearW {
        const self = self_(ctx);
        const w = try self.cpu.exec().loadLinear(name);
        errdefer self.cpu.exec().freeLinear(w);
        switch (w) {
            .f32 => return w, // stays on the CPU path
            .quant => |q| {
                if (self.be == null) return error.BackendUnavailable;
                var lin: QhipLinear = undefined;
                const rc = qhip_backend_load_linear(self.be, @intCast(@intFromEnum(q.ttype)), @intCast(q.rows),
                    @intCast(q.cols()), q.data.ptr, &lin);
                if (rc != 0) {
                    std.debug.print("hip backend: upload of '{s}' ({s}, {d} MiB) failed: {s}\n", .{
                        name, @tagName(q.ttype), q.data.len >> 20, qhip_error_string(rc),
                    });
                    return if (rc == 1) error.UnsupportedTensorType else error.OutOfMemory;
                }
                // the MMQ image of a prefill weight is built now, not inside a step
                _ = qhip_backend_prepare_linear(self.be, &lin);
                self.resident.append(self.alloc, .{ .host = q.data.ptr, .lin = lin }) catch {
                    qhip_backend_free_linear(self.be, &lin);
                    return error.OutOfMemory;
                };
                return w;
            },
        }
    }

    fn vFreeLinear(ctx: *anyopaque, w: backend.LinearW) void {
        const self = self_(ctx);
        switch (w) {
            .quant => |q| for (self.resident.items, 0..) |*r, i| {
                if (r.host == q.data.ptr) {
                    qhip_backend_free_linear(self.be, &r.lin);
                    _ = self.resident.swapRemove(i);
                    break;
                }
            },
            .f32 => {},
        }
        self.cpu.exec().freeLinear(w);
    }

    fn vMatvec(ctx: *anyopaque, out: backend.Buf, w: backend.LinearW, x: backend.Buf) void {
        const self = self_(ctx);
        const lin = switch (w) {
            .quant => |q| self.findDev(q.data.ptr),
            .f32 => null,
        } orelse return CpuBackend.vtable.matvec(&self.cpu, out, w, x);
        std.debug.assert(out.len >= @as(usize, @intCast(lin.rows)) and x.len >= @as(usize, @intCast(lin.cols)));
        self.finish("matvec", qhip_backend_matvec(self.be, out.ptr, lin, x.ptr), out);
        self.mvCheck(out, w, x, 1);
    }

    fn vMatvecPair(ctx: *anyopaque, out: backend.Buf, a: backend.LinearW, b: backend.LinearW, x: backend.Buf) void {
        const self = self_(ctx);
        const la = switch (a) {
            .quant => |q| self.findDev(q.data.ptr),
            .f32 => null,
        };
        const lb = switch (b) {
            .quant => |q| self.findDev(q.data.ptr),
            .f32 => null,
        };
        if (la == null or lb == null) return CpuBackend.vtable.matvecPair(&self.cpu, out, a, b, x);
        // one launch when the two device copies are adjacent and alike
        self.finish("matvecPair", qhip_backend_matvec_pair(self.be, out.ptr, la.?, lb.?, x.ptr), out);
    }

    fn vMatvecBatchK(ctx: *anyopaque, out: backend.Buf, w: backend.LinearW, xK: backend.Buf, k: usize) void {
        const self = self_(ctx);
        const lin = switch (w) {
            .quant => |q| self.findDev(q.data.ptr),
            .f32 => null,
        } orelse return CpuBackend.vtable.matvecBatchK(&self.cpu, out, w, xK, k);
        self.finish("matvecBatchK", qhip_backend_matvec_batch_k(self.be, out.ptr, lin, xK.ptr, @intCast(k)), out);
        self.mvCheck(out, w, xK, k);
    }

    fn vDequantRow(ctx: *anyopaque, dst: backend.Buf, w: gguf.QuantRow, row: usize) void {
        const self = self_(ctx);
        const lin = self.findDev(w.data.ptr) orelse return CpuBackend.vtable.dequantRow(&self.cpu, dst, w, row);
        self.finish("dequantRow", qhip_backend_dequant_row(self.be, dst.ptr, lin, @intCast(row)), dst);
    }

    fn dAllocScratch(ctx: *anyopaque, max_cols: usize) anyerror!void {
        return dAllocScratchK(ctx, max_cols, 1);
    }

    fn dAllocScratchK(ctx: *anyopaque, max_cols: usize, k: usize) anyerror!void {
        const self = self_(ctx);
        try CpuBackend.vtable.allocScratchK(&self.cpu, max_cols, k);
        const rc = qhip_backend_alloc_scratch_k(self.be, @intCast(max_cols), @intCast(k));
        if (rc != 0) {
            std.debug.print("hip backend: activation scratch: {s}\n", .{qhip_error_string(rc)});
            return error.OutOfMemory;
        }
    }

    fn dFreeScratch(ctx: *anyopaque) void {
        const self = self_(ctx);
        qhip_backend_free_scratch(self.be);
        freePinned(self);
        CpuBackend.vtable.freeScratch(&self.cpu);
    }

    /// Pinned host memory mapped into the GPU: the CPU slots use it as host
    /// memory, the HIP kernels through the mapping.
    fn dAllocBuf(ctx: *anyopaque, len: usize) anyerror!backend.Buf {
        const self = self_(ctx);
        var p: ?*anyopaque = null;
        const rc = hipHostMalloc(&p, @max(len, 1) * @sizeOf(f32), hipHostMallocMapped | hipHostMallocCoherent);
        if (rc != 0 or p == null) return error.OutOfMemory;
        errdefer _ = hipHostFree(p);
        try self.pinned.append(self.alloc, p.?);
        return .{ .ptr = @ptrCast(@alignCast(p.?)), .len = len };
    }

    fn dStepBegin(ctx: *anyopaque, pos: u32) void {
        const self = self_(ctx);
        qhip_backend_step_begin(self.be, pos);
        CpuBackend.vtable.stepBegin(&self.cpu, pos);
    }

    fn dStepEnd(ctx: *anyopaque) void {
        const self = self_(ctx);
        qhip_backend_step_end(self.be);
        CpuBackend.vtable.stepEnd(&self.cpu);
    }

    fn vName(ctx: *anyopaque) []const u8 {
        const self = self_(ctx);
        return if (self.be) |b| std.mem.span(qhip_backend_name(b)) else "hip (no device)";
    }

    /// backend.zig:494-495: the device, the bytes placed and the switches in
    /// use (the string is the library's, valid until the next call).
    fn vDescribe(ctx: *anyopaque) []const u8 {
        const self = self_(ctx);
        return if (self.be) |b| std.mem.span(qhip_backend_describe(b)) else "hip (no device)";
    }

    /// The library's device-timed slot table, then the CPU backend's table
    /// for the matvecs that stayed on the CPU (`.f32` weights).
    fn printDeviceTable(self: *HipBackend) void {
        const b = self.be orelse return;
        const n = qhip_backend_prof_report(b, null, 0);
        if (n <= 0) return;
        const text = self.alloc.alloc(u8, @intCast(n + 1)) catch return;
        defer self.alloc.free(text);
        _ = qhip_backend_prof_report(b, text.ptr, n + 1);
        std.debug.print("{s}", .{text[0..@intCast(n)]});
    }

    fn vReportProfile(ctx: *anyopaque) void {
        const self = self_(ctx);
        self.printDeviceTable();
        CpuBackend.vtable.reportProfile(&self.cpu);
    }

    fn vProfReport(ctx: *anyopaque) void {
        const self = self_(ctx);
        self.printDeviceTable();
        CpuBackend.vtable.profReport(&self.cpu);
    }

    /// The CPU backend's table with the quantized-matvec slots replaced.  The
    /// `Exec` context is the embedded CPU backend, so every other slot runs as
    /// it does in a CPU run; the slots above find their HipBackend from it.
    pub const vtable: backend.Exec.VTable = blk: {
        var vt = CpuBackend.vtable;
        vt.loadLinear = vLoadLinear;
        vt.freeLinear = vFreeLinear;
        vt.matvec = vMatvec;
        vt.matvecPair = vMatvecPair;
        vt.matvecBatchK = vMatvecBatchK;
        vt.dequantRow = vDequantRow;
        vt.allocScratch = dAllocScratch;
        vt.allocScratchK = dAllocScratchK;
        vt.freeScratch = dFreeScratch;
        vt.allocBuf = dAllocBuf;
        vt.stepBegin = dStepBegin;
        vt.stepEnd = dStepEnd;
        vt.name = vName;
        vt.describe = vDescribe;
        vt.reportProfile = vReportProfile;
        vt.profReport = vProfReport;
        break :blk vt;
    };
};
