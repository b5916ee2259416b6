'use strict';
// Mirrors the reference's tests/api/context.test.ts, tensor.test.ts: same
// cases, same expected values and error patterns.
const W = require('../../wgpu-executorch_amd/js');
const { describe, it, expect } = require('./harness');
const { WgpuExecutionContext, Tensor, MAX_NDIM, GPUBufferUsage } = W;
let cached = null;
async function setupGPU() { if (!cached) cached = await W.requestDevice(global.WGX_DEVICE_INDEX); return cached; }

describe('WgpuExecutionContext', () => {
  it('allocates storage buffers', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const buf = ctx.storageBuffer(256);
    expect(buf.size).toBeGreaterThanOrEqual(256);
    expect(buf.usage & GPUBufferUsage.STORAGE).toBeTruthy();
    ctx.destroy();
  });
  it('aligns storage buffer size to 4 bytes', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(ctx.storageBuffer(1).size).toBe(4);
    ctx.destroy();
  });
  it('creates tensors with owned buffers', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const t = ctx.tensor('float32', [2, 3]);
    expect(t.shape).toEqual([2, 3]);
    expect(t.byteLength).toBe(24);
    ctx.destroy();
  });
  it('copy() validates COPY_SRC on source', async () => {
    const device = await setupGPU();
    const ctx = new WgpuExecutionContext(device);
    const srcBuf = device.createBuffer({ size: 16, usage: GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_DST });
    const dst = ctx.tensor('float32', [4]);
    const src = new Tensor('float32', [4], device, srcBuf);
    expect(() => ctx.copy(src, dst)).toThrow(/COPY_SRC/);
    srcBuf.destroy();
    ctx.destroy();
  });
  it('copy() validates COPY_DST on destination', async () => {
    const device = await setupGPU();
    const ctx = new WgpuExecutionContext(device);
    const src = ctx.tensor('float32', [4]);
    const dstBuf = device.createBuffer({ size: 16, usage: GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_SRC });
    const dst = new Tensor('float32', [4], device, dstBuf);
    expect(() => ctx.copy(src, dst)).toThrow(/COPY_DST/);
    dstBuf.destroy();
    ctx.destroy();
  });
  it('copy() validates destination >= source size', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(() => ctx.copy(ctx.tensor('float32', [4]), ctx.tensor('float32', [2]))).toThrow(/< source/);
    ctx.destroy();
  });
  it('copy() + submit() transfers data between buffers', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const src = ctx.tensor('float32', [4]);
    const dst = ctx.tensor('float32', [4]);
    src.setData(new Float32Array([1, 2, 3, 4]));
    ctx.copy(src, dst);
    ctx.submit();
    await ctx.sync();
    expect(Array.from(new Float32Array(await dst.getData()))).toEqual([1, 2, 3, 4]);
    ctx.destroy();
  }, { gpu: true });
  it('destroy() prevents further use', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    ctx.destroy();
    expect(() => ctx.storageBuffer(16)).toThrow(/destroyed/);
  });
  it('destroy() is idempotent', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    ctx.destroy();
    expect(() => ctx.destroy()).not.toThrow();
  });
  it('submit() with no commands is a no-op', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(() => ctx.submit()).not.toThrow();
    ctx.destroy();
  });
  it('sync() resolves after submit()', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const src = ctx.tensor('float32', [4]).setData(new Float32Array([1, 2, 3, 4]));
    ctx.copy(src, ctx.tensor('float32', [4]));
    ctx.submit();
    await expect(ctx.sync()).resolves.toBeUndefined();
    ctx.destroy();
  }, { gpu: true });
  it('sync() with no prior submit() resolves', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    await expect(ctx.sync()).resolves.toBeUndefined();
    ctx.destroy();
  });
  it('sync() on destroyed context throws', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    ctx.destroy();
    await expect(ctx.sync()).rejects.toThrow(/destroyed/);
  });
  it('submit() of a command whose buffer was destroyed fails instead of touching it', async () => {
    const device = await setupGPU();
    const ctx = new WgpuExecutionContext(device);
    const buf = device.createBuffer({ size: 16, usage: GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_SRC | GPUBufferUsage.COPY_DST });
    const src = new Tensor('float32', [4], device, buf);
    ctx.copy(src, ctx.tensor('float32', [4]));
    buf.destroy();
    expect(() => ctx.submit()).toThrow(/destroyed buffer/);
    ctx.destroy();
  }, { gpu: true });
});

describe('Tensor', () => {
  it('creates a tensor with valid shape', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const t = ctx.tensor('float32', [2, 3]);
    expect(t.shape).toEqual([2, 3]);
    expect(t.numel).toBe(6);
    expect(t.byteLength).toBe(24);
    expect(t.dtype).toBe('float32');
    ctx.destroy();
  });
  it('rejects rank > MAX_NDIM', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(() => ctx.tensor('float32', new Array(MAX_NDIM + 1).fill(1))).toThrow(/exceeds maximum rank/);
    ctx.destroy();
  });
  it('rejects zero / negative / non-integer dimensions', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(() => ctx.tensor('float32', [0, 3])).toThrow(/positive integers/);
    expect(() => ctx.tensor('float32', [-1, 3])).toThrow(/positive integers/);
    expect(() => ctx.tensor('float32', [1.5, 3])).toThrow(/positive integers/);
    ctx.destroy();
  });
  it('rejects buffer too small', async () => {
    const device = await setupGPU();
    const buf = device.createBuffer({ size: 4, usage: GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_DST | GPUBufferUsage.COPY_SRC });
    expect(() => new Tensor('float32', [2, 3], device, buf)).toThrow(/< required/);
    buf.destroy();
  });
  it('rejects buffer without STORAGE usage', async () => {
    const device = await setupGPU();
    const buf = device.createBuffer({ size: 24, usage: GPUBufferUsage.COPY_DST | GPUBufferUsage.COPY_SRC });
    expect(() => new Tensor('float32', [2, 3], device, buf)).toThrow(/STORAGE flag/);
    buf.destroy();
  });
  it('setData uploads TypedArray / ArrayBuffer data and getData reads it back', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const t = ctx.tensor('float32', [2, 3]);
    t.setData(new Float32Array([1, 2, 3, 4, 5, 6]));
    expect(Array.from(new Float32Array(await t.getData()))).toEqual([1, 2, 3, 4, 5, 6]);
    const u = ctx.tensor('float32', [2, 2]);
    u.setData(new Float32Array([1, 2, 3, 4]).buffer);
    expect(Array.from(new Float32Array(await u.getData()))).toEqual([1, 2, 3, 4]);
    ctx.destroy();
  });
  it('setData writes a prefix when the source is smaller than the tensor', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const t = ctx.tensor('float32', [2, 3]);
    t.setData(new Float32Array([1, 2, 3, 4, 5, 6]));
    t.setData(new Float32Array([7, 8]));
    expect(Array.from(new Float32Array(await t.getData()))).toEqual([7, 8, 3, 4, 5, 6]);
    ctx.destroy();
  });
  it('setData rejects source larger than tensor', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    expect(() => ctx.tensor('float32', [2, 3]).setData(new Float32Array(8))).toThrow(/pass a view/);
    ctx.destroy();
  });
  it('setData rejects buffer without COPY_DST', async () => {
    const device = await setupGPU();
    const buf = device.createBuffer({ size: 24, usage: GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_SRC });
    const t = new Tensor('float32', [2, 3], device, buf);
    expect(() => t.setData(new Float32Array([1, 2, 3, 4, 5, 6]))).toThrow(/COPY_DST/);
    buf.destroy();
  });
  it('handles unaligned byte sizes in setData and getData', async () => {
    const ctx = new WgpuExecutionContext(await setupGPU());
    const t = ctx.tensor('uint8', [3]);
    t.setData(new Uint8Array([7, 42, 99]));
    expect(Array.from(new Uint8Array(await t.getData()))).toEqual([7, 42, 99]);
    ctx.destroy();
  });
  it('float16 helpers round to nearest even', async () => {
    expect(W.toHalf(1 + Math.pow(2, -11))).toBe(0x3c00);
    expect(W.toHalf(1 + 3 * Math.pow(2, -11))).toBe(0x3c02);
    expect(W.toHalf(65520)).toBe(0x7c00);
    expect(W.fromHalf(0x3555)).toBeCloseTo(0.33325, 5);
  });
});
