'use strict';
/**
 * Node host layer of wgpu-executorch_amd: the reference's public API for the
 * GEMM-shaped hot path (src/tensor.ts, src/context.ts, src/shader.ts,
 * src/program.ts, src/shaders/index.ts), executing through libwgx (the
 * MI355X C-ABI in include/wgx.h) via the N-API addon wgx_napi.node.
 *
 * Written as ES2019 CommonJS because this image's Node is v12 and has no
 * TypeScript compiler; index.d.ts carries the types.  Validation and error
 * texts follow the reference drivers so code and tests written against the
 * reference behave the same; the C library re-validates every record
 * against the buffers it owns, so no launch can address memory outside them.
 */
const path = require('path');
const native = require(path.join(__dirname, 'wgx_napi.node'));

// ------------------------------------------------------------------ tensor.ts

/** GPUBufferUsage flags (WebGPU values). */
const GPUBufferUsage = Object.freeze({
  MAP_READ: 0x1, MAP_WRITE: 0x2, COPY_SRC: 0x4, COPY_DST: 0x8, INDEX: 0x10, VERTEX: 0x20,
  UNIFORM: 0x40, STORAGE: 0x80, INDIRECT: 0x100, QUERY_RESOLVE: 0x200,
});

/** src/tensor.ts:23 */
const MAX_NDIM = 8;

/** src/tensor.ts:26-30, plus bfloat16. */
const DTYPE_BYTESIZE = Object.freeze({
  float32: 4, float16: 2, float64: 8, int32: 4, int64: 8, int8: 1, uint8: 1, bool: 1, bfloat16: 2,
});
const DTYPE_CODE = Object.freeze({
  float32: 0, float16: 1, int32: 2, int8: 3, uint8: 4, bool: 5, float64: 6, int64: 7, bfloat16: 8,
});

const STORAGE_BUFFER_USAGE = GPUBufferUsage.STORAGE | GPUBufferUsage.COPY_SRC | GPUBufferUsage.COPY_DST;
const UNIFORM_BUFFER_USAGE = GPUBufferUsage.UNIFORM | GPUBufferUsage.COPY_DST;

/**
 * A device allocation (the GPUBuffer stand-in).  `ptr` is the HIP device
 * address; `view(offset, size)` makes a sub-range that tensors can wrap
 * (used for memory-plan pools carved out of one allocation).
 */
class WgxBuffer {
  constructor(device, ptr, size, usage, base) {
    this._device = device;
    this.ptr = ptr;
    this.size = size;
    this.usage = usage;
    this._base = base || null;
    this._destroyed = false;
  }

  view(offset, size) {
    return new WgxBuffer(this._device, this.ptr + offset, size, this.usage, this._base || this);
  }

  destroy() {
    if (this._destroyed || this._base || this.ptr === 0) return;
    this._destroyed = true;
    native.free(this._device._h, this.ptr);
  }
}

/**
 * One GPU (the GPUDevice stand-in).  It owns the device-wide buffer
 * registry and the queue (one HIP stream): every WgpuExecutionContext made
 * on it submits to that queue in order.
 */
class WgxDevice {
  constructor(index) {
    this._h = native.ctxCreate(index);
    const info = native.ctxInfo(this._h);
    this.index = index;
    this.arch = info.arch;
    this.features = new Set(['shader-f16']);
    const self = this;
    this.queue = {
      writeBuffer(buffer, offset, data, dataOffset, size) {
        const ab = data instanceof ArrayBuffer ? data : data.buffer;
        const base = data instanceof ArrayBuffer ? 0 : data.byteOffset;
        native.write(self._h, buffer.ptr + (offset || 0), ab, base + (dataOffset || 0),
          size === undefined ? ab.byteLength - base - (dataOffset || 0) : size);
      },
      /** Settles when the work submitted so far is done (waited off the JS thread). */
      onSubmittedWorkDone() {
        return native.syncAsync(self._h);
      },
    };
  }

  /** device.createBuffer({size, usage}): a device allocation the caller owns. */
  createBuffer(desc) {
    const size = Math.max(4, Math.ceil(desc.size / 4) * 4);
    const ptr = native.alloc(this._h, size, desc.usage);
    return new WgxBuffer(this, ptr, desc.size, desc.usage);
  }

  destroy() {
    if (this._h) native.ctxDestroy(this._h);
    this._h = null;
  }
}

/** Opens GPU `index` (HIP device ordinal); -1 gives a host-only validation device. */
async function requestDevice(index) {
  return new WgxDevice(index === undefined ? 0 : index);
}

function createDevice(index) {
  return new WgxDevice(index === undefined ? 0 : index);
}

/** A non-owning tensor view (src/tensor.ts:43-159). */
class Tensor {
  constructor(dtype, shape, device, buffer) {
    if (shape.length > MAX_NDIM) {
      throw new Error(`Tensor rank ${shape.length} exceeds maximum rank of ${MAX_NDIM}`);
    }
    if (shape.some((dim) => dim <= 0 || !Number.isInteger(dim))) {
      throw new Error('Tensor dimensions must be positive integers');
    }
    this._dtype = dtype;
    this._shape = shape;
    this._numel = shape.reduce((a, b) => a * b, 1);
    this._buffer = buffer;
    this._device = device;
    const requiredBytes = this._numel * DTYPE_BYTESIZE[dtype];
    if (buffer.size < requiredBytes) {
      throw new Error(`GPUBuffer size (${buffer.size}B) < required (${requiredBytes}B)`);
    }
    if ((buffer.usage & GPUBufferUsage.STORAGE) === 0) {
      throw new Error('GPUBuffer must have GPUBufferUsage.STORAGE flag');
    }
  }

  get dtype() { return this._dtype; }
  get numel() { return this._numel; }
  get shape() { return this._shape; }
  get buffer() { return this._buffer; }
  get device() { return this._device; }
  get byteLength() { return this._numel * DTYPE_BYTESIZE[this._dtype]; }

  /** {ptr, dtype, shape} for the native records. */
  _c() {
    return { ptr: this._buffer.ptr, dtype: DTYPE_CODE[this._dtype], shape: this._shape };
  }

  /** src/tensor.ts:115-135: prefix write, padded to 4 bytes. */
  setData(src) {
    const byteLength = this.byteLength;
    if ((this._buffer.usage & GPUBufferUsage.COPY_DST) === 0) {
      throw new Error('setData: buffer missing COPY_DST usage');
    }
    if (src.byteLength > byteLength) {
      throw new Error(`setData: source ${src.byteLength}B > tensor ${byteLength}B; pass a view`);
    }
    const alignedSize = Math.min(Math.ceil(src.byteLength / 4) * 4, this._buffer.size);
    const bytes = new Uint8Array(Math.ceil(src.byteLength / 4) * 4);
    bytes.set(src instanceof ArrayBuffer
      ? new Uint8Array(src, 0, src.byteLength)
      : new Uint8Array(src.buffer, src.byteOffset, src.byteLength));
    native.write(this._device._h, this._buffer.ptr, bytes.buffer, 0, alignedSize);
    return this;
  }

  /** src/tensor.ts:142-158: waits for submitted work, resolves the bytes. */
  async getData() {
    return native.read(this._device._h, this._buffer.ptr, this.byteLength);
  }
}

// ------------------------------------------------------------------ context.ts

/** Execution context (src/context.ts:17-390). */
class WgpuExecutionContext {
  constructor(device) {
    this._device = device;
    this._h = native.ctxCreateShared(device._h);
    this._destroyed = false;
  }

  get device() { return this._device; }

  _assertNotDestroyed() {
    if (this._destroyed) throw new Error('WgpuExecutionContext is destroyed');
  }

  destroy() {
    if (this._destroyed) return;
    this._destroyed = true;
    native.ctxDestroy(this._h);  // frees every buffer this context allocated
  }

  storageBuffer(size) {
    this._assertNotDestroyed();
    const alignedSize = Math.max(4, Math.ceil(size / 4) * 4);
    const ptr = native.alloc(this._h, alignedSize, STORAGE_BUFFER_USAGE);
    return new WgxBuffer(this._device, ptr, alignedSize, STORAGE_BUFFER_USAGE);
  }

  /**
   * Parameters reach the kernels by value here, so a uniform buffer is a
   * host-side record of its bytes (kept for API compatibility).
   */
  uniformBuffer(data) {
    this._assertNotDestroyed();
    const bytes = data instanceof ArrayBuffer ? data.slice(0) : data.buffer.slice(data.byteOffset, data.byteOffset + data.byteLength);
    const buf = new WgxBuffer(this._device, 0, Math.max(16, Math.ceil(bytes.byteLength / 4) * 4), UNIFORM_BUFFER_USAGE);
    buf.data = bytes;
    return buf;
  }

  tensor(dtype, shape, buffer) {
    this._assertNotDestroyed();
    if (buffer !== undefined) return new Tensor(dtype, shape, this._device, buffer);
    const numel = shape.reduce((a, b) => a * b, 1);
    return new Tensor(dtype, shape, this._device, this.storageBuffer(numel * DTYPE_BYTESIZE[dtype]));
  }

  /** Raw WebGPU dispatch descriptors have no equivalent here (no WGSL pipelines). */
  addDispatch() {
    this._assertNotDestroyed();
    throw new Error('addDispatch: WebGPU pipelines do not exist on the MI355X backend; record operators with recordShader');
  }

  copy(src, dst) {
    this._assertNotDestroyed();
    if ((src.buffer.usage & GPUBufferUsage.COPY_SRC) === 0) {
      throw new Error('copy: source buffer missing COPY_SRC usage');
    }
    if ((dst.buffer.usage & GPUBufferUsage.COPY_DST) === 0) {
      throw new Error('copy: destination buffer missing COPY_DST usage');
    }
    if (dst.byteLength < src.byteLength) {
      throw new Error(`copy: destination (${dst.byteLength}B) < source (${src.byteLength}B)`);
    }
    // src/context.ts:182-189: the copy is padded to whole 4-byte words.  A
    // buffer this backend carves out of a larger allocation (a view) may end
    // at the tensor's last byte, and the bytes after it then belong to
    // another tensor: the padding stops at the end of either buffer.
    const padded = Math.ceil(src.byteLength / 4) * 4;
    native.recordCopy(this._h, dst.buffer.ptr, src.buffer.ptr, Math.min(padded, src.buffer.size, dst.buffer.size));
    return this;
  }

  recordShader(shader, args) {
    this._assertNotDestroyed();
    shader.recordIn(this, args);
    return this;
  }

  /**
   * src/context.ts:219-317.  Memory-plan pools become views into ONE device
   * allocation (256-byte aligned offsets) and constants into one weights
   * allocation, instead of one buffer per pool / per constant.
   */
  recordProgram(program, weights, args, options) {
    this._assertNotDestroyed();
    const fuse = !(options && options.fuse === false);
    const useViews = !(options && options.views === false);
    const numInputs = program.inputIds.length;
    const numOutputs = program.outputIds.length;
    if (args.length !== numInputs + numOutputs) {
      throw new Error(`program: expected ${numInputs + numOutputs} args, got ${args.length}`);
    }
    const align = (n) => Math.ceil(n / 256) * 256;

    // pools -> one slab
    const poolOffset = new Map();
    let poolBytes = 0;
    for (const pool of program.memoryPlan.pools) {
      poolOffset.set(pool.id, { off: poolBytes, size: Math.max(4, Math.ceil(pool.size / 4) * 4) });
      poolBytes += align(Math.max(4, pool.size));
    }
    const poolSlab = poolBytes > 0 ? this.storageBuffer(poolBytes) : null;

    // constants -> one slab (each constant realigned to 256 bytes)
    const constOffset = new Map();
    let constBytes = 0;
    program.values.forEach((v, i) => {
      if (v.type === 'tensor' && v.weightsOffset !== undefined && v.weightsLength !== undefined) {
        constOffset.set(i, constBytes);
        constBytes += align(Math.max(4, v.weightsLength));
      }
    });
    const constSlab = constBytes > 0 ? this.storageBuffer(constBytes) : null;

    // zero-copy cat / split / view_copy groups -> one slab of their own
    const views = useViews ? planViews(program) : { place: new Map(), groupBytes: new Map(), elided: new Set() };
    const groupOffset = new Map();
    let groupBytes = 0;
    for (const [root, bytes] of views.groupBytes) {
      groupOffset.set(root, groupBytes);
      groupBytes += align(Math.max(4, bytes));
    }
    const groupSlab = groupBytes > 0 ? this.storageBuffer(groupBytes) : null;

    const tensors = new Map();
    program.values.forEach((v, i) => {
      if (v.type !== 'tensor') return;
      let buffer;
      if (views.place.has(i)) {
        const p = views.place.get(i);
        buffer = groupSlab.view(groupOffset.get(p.root) + p.off, valueBytes(v));
      } else if (v.weightsOffset !== undefined && v.weightsLength !== undefined) {
        buffer = constSlab.view(constOffset.get(i), Math.max(4, Math.ceil(v.weightsLength / 4) * 4));
      } else if (v.memObjId !== undefined) {
        if (!poolOffset.has(v.memObjId)) {
          throw new Error(`program: no memory pool ${v.memObjId} for value ${i}`);
        }
        const p = poolOffset.get(v.memObjId);
        buffer = poolSlab.view(p.off, p.size);
      } else {
        const numel = v.shape.reduce((a, b) => a * b, 1);
        buffer = this.storageBuffer(numel * DTYPE_BYTESIZE[v.dtype]);
      }
      tensors.set(i, this.tensor(v.dtype, v.shape, buffer));
    });

    // Program inputs and outputs bound to the caller's tensors (no copy in or
    // out; this build's own pass, switched off with {bindIO: false}): an input
    // that no op writes is read in place; an output that exactly one op
    // writes is written in place by that op.  Each bound tensor must have the
    // value's dtype and size, and the caller's inputs and outputs must not
    // share memory.  The copies' semantics hold: the chain reads the caller's
    // input as it is at submit time, and nothing else writes the output.
    const bound = new Set();
    if (!(options && options.bindIO === false)) {
      const writers = new Map();
      for (const op of program.chain) {
        for (const id of opOutputs(op, program.values)) writers.set(id, (writers.get(id) || 0) + 1);
      }
      const ins = args.slice(0, numInputs), outs = args.slice(numInputs);
      // bound tensors must not share memory across the input / output
      // boundary, and two outputs must not share memory either (the
      // producer of one would overwrite the other while later ops still
      // read it)
      const ioClash = ins.some((a) => a instanceof Tensor && outs.some((o) => o instanceof Tensor && overlaps(a, o))) ||
        outs.some((o, i) => o instanceof Tensor && outs.some((p, j) => j !== i && p instanceof Tensor && overlaps(o, p)));
      const fits = (t, id) => t instanceof Tensor && t.dtype === program.values[id].dtype &&
        t.byteLength === valueBytes(program.values[id]);
      const once = (ids) => (id) => ids.filter((x) => x === id).length === 1;
      const inOnce = once(program.inputIds), outOnce = once(program.outputIds);
      if (!ioClash) {
        program.inputIds.forEach((id, i) => {
          if (fits(ins[i], id) && inOnce(id) && !writers.has(id) && !program.outputIds.includes(id) &&
              !views.place.has(id)) {
            tensors.set(id, ins[i]);
            bound.add(id);
          }
        });
        program.outputIds.forEach((id, i) => {
          if (fits(outs[i], id) && outOnce(id) && writers.get(id) === 1 && !program.inputIds.includes(id) &&
              !views.place.has(id) && !constOffset.has(id)) {
            tensors.set(id, outs[i]);
            bound.add(id);
          }
        });
      }
    }

    // weights: one staging image of the constant slab, one upload
    if (constSlab) {
      const staging = new Uint8Array(constBytes);
      const src = weights instanceof ArrayBuffer ? new Uint8Array(weights)
        : new Uint8Array(weights.buffer, weights.byteOffset, weights.byteLength);
      program.values.forEach((v, i) => {
        if (constOffset.has(i)) {
          staging.set(src.subarray(v.weightsOffset, v.weightsOffset + v.weightsLength), constOffset.get(i));
        }
      });
      native.write(this._device._h, constSlab.ptr, staging.buffer, 0, constBytes);
    }

    let fused = new Map();
    if (fuse) {
      const triples = siluTriples(program);
      // The fused launch writes the last tensor of the group (y, or z with a
      // residual) while it reads the convolution's input, weight and bias
      // (and the residual, element for element).  A memory plan may give that
      // output the space of an input that is dead after it (the unfused ops
      // never read it then), so such an output, when it is not part of a view
      // group, moves to memory of its own: one buffer for all of them.
      const outOf = (t) => (t.add ? t.add.z : t.y);
      const clash = (t) => {
        const to = tensors.get(outOf(t));
        if (convReads(program, t.k, tensors).some((r) => overlaps(r, to))) return true;
        if (!t.add) return false;
        const tr = tensors.get(t.add.r);
        return tr.buffer.ptr !== to.buffer.ptr && overlaps(tr, to);  // the same memory is fine
      };
      const moved = triples.filter((t) => !views.place.has(outOf(t)) && clash(t));
      const movedBytes = moved.reduce((n, t) => n + align(Math.max(4, tensors.get(outOf(t)).byteLength)), 0);
      if (movedBytes > 0) {
        const slab = this.storageBuffer(movedBytes);
        let at = 0;
        for (const t of moved) {
          const to = tensors.get(outOf(t));
          tensors.set(outOf(t), this.tensor(to.dtype, to.shape, slab.view(at, to.byteLength)));
          at += align(Math.max(4, to.byteLength));
        }
      }
      for (const t of triples) {
        if (clash(t)) continue;
        const fargs = resolveArgs(program.chain[t.k], program.values, tensors);
        fargs.pop();
        if (t.add) {
          fargs.push(tensors.get(t.add.r), t.add.convScale, t.add.residualScale, tensors.get(t.add.z));
          fused.set(t.k, { shader: shaders.convolutionSiluAdd, args: fargs, ops: 4, y: t.y });
        } else {
          fargs.push(tensors.get(t.y));
          fused.set(t.k, { shader: shaders.convolutionSilu, args: fargs, ops: 3 });
        }
      }
    }

    for (let i = 0; i < numInputs; i++) {
      const src = args[i];
      const dst = tensors.get(program.inputIds[i]);
      if (!(src instanceof Tensor)) continue;
      if (dst === undefined) throw new Error(`program: no tensor for input value ${program.inputIds[i]}`);
      if (bound.has(program.inputIds[i])) continue;  // the chain reads the caller's tensor itself
      this.copy(src, dst);
    }

    for (let k = 0; k < program.chain.length; k++) {
      if (views.elided.has(k)) continue;  // its output already is its inputs' bytes
      const f = fused.get(k);
      if (f !== undefined) {  // conv -> sigmoid -> mul (-> add) as one convolution launch
        if (f.ops === 4) {
          try {
            this.recordShader(f.shader, f.args);
          } catch (e) {
            // a convolution whose kernel has no residual epilogue: conv+SiLU
            // into the product, then the add as an op of its own -- or, when
            // the memory plan gives the product the space of something the
            // convolution reads (the unfused chain writes it only later), the
            // four ops as they stand
            if (!/residual is supported/.test(e.message)) throw e;
            const ty = tensors.get(f.y);
            if (convReads(program, k, tensors).some((r) => overlaps(r, ty))) {
              for (let q = k; q < k + 3; q++) {
                const op = program.chain[q];
                this.recordShader(shaderRegistry[op.name], resolveArgs(op, program.values, tensors));
              }
            } else {
              const sargs = f.args.slice(0, 9);
              sargs.push(ty);
              this.recordShader(shaders.convolutionSilu, sargs);
            }
            const addOp = program.chain[k + 3];
            this.recordShader(shaderRegistry[addOp.name], resolveArgs(addOp, program.values, tensors));
          }
        } else {
          this.recordShader(f.shader, f.args);
        }
        k += f.ops - 1;
        continue;
      }
      const op = program.chain[k];
      const shader = shaderRegistry[op.name];
      if (!shader) throw new Error(`program: unknown operator '${op.name}'`);
      this.recordShader(shader, resolveArgs(op, program.values, tensors));
    }

    for (let i = 0; i < numOutputs; i++) {
      const src = tensors.get(program.outputIds[i]);
      const dst = args[numInputs + i];
      if (!(dst instanceof Tensor)) throw new Error(`program: output ${i} must be a Tensor`);
      if (src === undefined) throw new Error(`program: no tensor for output value ${program.outputIds[i]}`);
      if (bound.has(program.outputIds[i])) continue;  // its producer wrote the caller's tensor
      this.copy(src, dst);
    }
    return this;
  }

  submit() {
    this._assertNotDestroyed();
    native.submit(this._h);
  }

  /**
   * src/context.ts:377-380: a Promise that settles when the work submitted
   * so far is done.  The wait runs on a libuv worker, so the JS thread keeps
   * running (and may record the next frame) meanwhile.
   */
  async sync() {
    this._assertNotDestroyed();
    await native.syncAsync(this._h);
  }

  reset() {
    this._assertNotDestroyed();
    native.reset(this._h);
  }

  /** Extras of this backend: replay through a HIP graph (default) or eagerly. */
  setGraphMode(enabled) { native.setGraphMode(this._h, enabled ? 1 : 0); }

  /** Mean device time of `reps` back-to-back submits, HIP events on the queue. */
  timeSubmits(reps) { return native.timeSubmits(this._h, reps); }

  /** Kernel chosen by the most recent record. */
  get lastKernel() { return native.ctxInfo(this._h).lastKernel; }

  get commandCount() { return native.ctxInfo(this._h).commandCount; }
}

// ------------------------------------------------------------------ program.ts

/** src/program.ts:188-224 */
function resolveArgs(op, values, tensors) {
  return op.args.map((idx) => {
    const v = values[idx];
    switch (v.type) {
      case 'tensor': {
        const t = tensors.get(idx);
        if (t === undefined) throw new Error(`program: no tensor for value ${idx} referenced by '${op.name}'`);
        return t;
      }
      case 'scalar':
        return v.value;
      case 'list':
        return v.items.slice();
      case 'tensorlist':
        return v.items.map((j) => {
          const item = values[j];
          if (!item || item.type !== 'tensor') {
            throw new Error(`program: tensorlist item ${j} is not a tensor (${op.name})`);
          }
          const t = tensors.get(j);
          if (t === undefined) throw new Error(`program: no tensor for value ${j} referenced by '${op.name}'`);
          return t;
        });
      case 'null':
        return undefined;
      default:
        return undefined;
    }
  });
}

/**
 * The converter's consistency rules for a program and its weights
 * (utils/pte_to_program.py:421-475, same messages), for hosts that load
 * converted files.  One relaxation: the weights may be longer than the sum
 * of the declared constant lengths, since the float16 converter pads each
 * constant to a 4-byte offset (utils/convert_model_to_fp16.mjs:61-66) and
 * does not re-validate.  recordProgram itself keeps the reference's own
 * checks and messages (src/context.ts:219-317).
 */
function validateProgram(program, weightsByteLength) {
  const { values, chain } = program;
  let declared = 0;
  for (const v of values) if (v.type === 'tensor' && v.weightsLength !== undefined) declared += v.weightsLength;
  if (declared > weightsByteLength) {
    throw new Error(`Weights size mismatch: declared ${declared} bytes, actual ${weightsByteLength} bytes`);
  }
  chain.forEach((op, ci) => {
    for (const arg of op.args) {
      if (Number.isInteger(arg) && (arg < 0 || arg >= values.length)) {
        throw new Error(`chain[${ci}] '${op.name}' references values[${arg}] but only ${values.length} values exist`);
      }
    }
  });
  for (const [label, ids] of [['inputIds', program.inputIds], ['outputIds', program.outputIds]]) {
    for (const idx of ids) {
      if (idx < 0 || idx >= values.length) throw new Error(`${label} references values[${idx}] out of range`);
      if (values[idx].type !== 'tensor') {
        throw new Error(`${label} references values[${idx}] of type '${values[idx].type}', expected 'tensor'`);
      }
    }
  }
  const poolIds = new Set(program.memoryPlan.pools.map((p) => p.id));
  values.forEach((v, i) => {
    if (v.type === 'tensor' && v.memObjId !== undefined && !poolIds.has(v.memObjId)) {
      throw new Error(`values[${i}] has memObjId=${v.memObjId} but no matching pool in memoryPlan. ` +
        `Available pools: [${[...poolIds].sort((a, b) => a - b).join(', ')}]`);
    }
  });
  values.forEach((v, i) => {
    if (v.type === 'tensor' && v.weightsOffset !== undefined) {
      const end = v.weightsOffset + v.weightsLength;
      if (end > weightsByteLength) {
        throw new Error(`values[${i}] weights [${v.weightsOffset}:${end}] exceeds weights.bin size (${weightsByteLength})`);
      }
    }
  });
}

// ------------------------------------------------------------------ graph-level fusion

function valueBytes(v) {
  return v.shape.reduce((a, b) => a * b, 1) * DTYPE_BYTESIZE[v.dtype];
}

function overlaps(a, b) {
  return a.buffer.ptr < b.buffer.ptr + b.byteLength && b.buffer.ptr < a.buffer.ptr + a.byteLength;
}

/** How many times each value is read by the chain (program outputs count once). */
function useCounts(program) {
  const uses = new Map();
  const note = (id) => uses.set(id, (uses.get(id) || 0) + 1);
  for (const op of program.chain) {
    for (const a of op.args) {
      const v = program.values[a];
      if (!v) continue;
      if (v.type === 'tensor') note(a);
      else if (v.type === 'tensorlist') v.items.forEach(note);
    }
  }
  for (const id of program.outputIds) note(id);
  return uses;
}

/** Values an op writes: out-variant operators take their outputs last. */
function opOutputs(op, values) {
  const last = op.args[op.args.length - 1];
  const v = values[last];
  if (!v) return [];
  if (v.type === 'tensor') return [last];
  if (v.type === 'tensorlist') return v.items.slice();
  return [];
}

/** The tensors a convolution reads (input, weight, bias). */
function convReads(program, k, tensors) {
  const conv = program.chain[k];
  return [0, 1, 2].map((i) => conv.args[i])
    .filter((i) => program.values[i] && program.values[i].type === 'tensor')
    .map((i) => tensors.get(i));
}

/**
 * SiLU after a convolution, as exported graphs spell it: conv -> c,
 * sigmoid(c) -> s, mul(c, s) -> y, three consecutive ops.  When c and s are
 * read by nothing else (and are not program outputs) the convolution can
 * write SiLU(conv) straight into y, one launch instead of three and two
 * feature-map round trips fewer.  When the next op is aten.add.Tensor with y
 * as one operand (and y read by nothing else), the add joins too: the
 * depthwise kernels and the dense LDS-patch kernel add an output-shaped
 * residual in their epilogue (a convolution that another kernel runs is
 * recorded as conv+SiLU and the add, see recordProgram).  Returns {k, y,
 * add}: k the convolution's chain index, y the product, add null or {k, r, z,
 * convScale, residualScale} with z = the add's output = convScale * y +
 * residualScale * r.
 */
function siluTriples(program) {
  const { chain, values } = program;
  const uses = useCounts(program);
  const out = [];
  const same = (a, b) => a && b && a.type === 'tensor' && b.type === 'tensor' && a.dtype === b.dtype &&
    a.shape.length === b.shape.length && a.shape.every((d, i) => d === b.shape[i]);
  for (let k = 0; k + 2 < chain.length; k++) {
    const conv = chain[k], sig = chain[k + 1], mul = chain[k + 2];
    if (conv.name !== 'aten.convolution.default' || sig.name !== 'aten.sigmoid.default' ||
        mul.name !== 'aten.mul.Tensor' || sig.args.length !== 2 || mul.args.length !== 3) continue;
    const c = conv.args[conv.args.length - 1], s = sig.args[1], y = mul.args[2];
    if (sig.args[0] !== c || !((mul.args[0] === c && mul.args[1] === s) || (mul.args[0] === s && mul.args[1] === c))) continue;
    if (uses.get(c) !== 3 || uses.get(s) !== 2 || !same(values[c], values[y])) continue;
    const t = { k, y, add: null };
    // aten.add.Tensor(a, b, alpha) -> z right after, with y one operand and
    // read by nothing else: the residual epilogue
    const add = chain[k + 3];
    if (add && add.name === 'aten.add.Tensor' && add.args.length === 4 && uses.get(y) === 2 &&
        (add.args[0] === y) !== (add.args[1] === y)) {
      const r = add.args[0] === y ? add.args[1] : add.args[0];
      const av = values[add.args[2]];
      const alpha = av && av.type === 'scalar' ? Number(av.value) : 1;
      const transposed = values[conv.args[6]] && values[conv.args[6]].value;
      if (!transposed && Number.isFinite(alpha) && same(values[r], values[y]) && same(values[add.args[3]], values[y])) {
        t.add = { k: k + 3, r, z: add.args[3],
          convScale: add.args[1] === y ? alpha : 1, residualScale: add.args[1] === y ? 1 : alpha };
      }
    }
    out.push(t);
    k += t.add ? 3 : 2;
  }
  return out;
}

/**
 * Zero-copy concatenation, split and flat copies.  When every dimension
 * before the cat (split) dimension has size 1, a concatenation is its inputs
 * laid end to end and each piece of a split is a contiguous byte range of
 * its input; a view_copy, squeeze_copy, unsqueeze_copy or clone (without a
 * memory format) is its input's bytes unchanged.  If the producers of
 * the pieces write straight into the whole, such an op has nothing left to
 * do.  Each op ties its tensors together at fixed byte offsets (a union-find
 * with offsets); tied tensors form a group that gets memory of its own,
 * outside the memory-plan pools, whose sharing assumes the copies happen.
 * An op is taken only if, with it, every group still has exactly one writer
 * per byte (a tensor written by an op that still runs) and every tensor's
 * bytes are all written; otherwise its ties are undone and it runs as a copy.
 * Program inputs, outputs and constants never join a group.
 *
 * Returns place: value -> {root, off} (byte offset within the group),
 * groupBytes: root -> group size, elided: chain indices with nothing to do.
 */
// Copies whose output is their input's bytes unchanged (a clone without a
// memory format; the shape-only copies).
const FLAT_COPIES = new Set(['aten.view_copy.default', 'aten.clone.default', 'aten.squeeze_copy.dims',
  'aten.unsqueeze_copy.default']);

function planViews(program) {
  const { chain, values } = program;
  const producer = new Map();
  chain.forEach((op, k) => {
    for (const id of opOutputs(op, values)) producer.set(id, producer.has(id) ? -1 : k);
  });
  const fixed = new Set([...program.inputIds, ...program.outputIds]);
  const movable = (id) => {
    const v = values[id];
    return v && v.type === 'tensor' && v.weightsOffset === undefined && !fixed.has(id) &&
      producer.get(id) >= 0 && valueBytes(v) > 0;
  };

  let parent = new Map(), offset = new Map();
  const find = (id) => {
    let d = 0;
    while (parent.has(id)) { d += offset.get(id); id = parent.get(id); }
    return [id, d];
  };
  // a's bytes start `delta` bytes after b's
  const tie = (a, b, delta) => {
    const [ra, da] = find(a), [rb, db] = find(b);
    if (ra === rb) return da === db + delta;
    parent.set(ra, rb);
    offset.set(ra, db + delta - da);
    return true;
  };
  const members = new Set();
  const elided = new Set();
  const consistent = () => {
    const groups = new Map();
    for (const id of members) {
      const [r, d] = find(id);
      if (!groups.has(r)) groups.set(r, []);
      groups.get(r).push({ id, lo: d, hi: d + valueBytes(values[id]) });
    }
    for (const list of groups.values()) {
      if (list.some((m) => values[m.id].dtype !== values[list[0].id].dtype)) return false;
      const writers = list.filter((m) => !elided.has(producer.get(m.id))).sort((a, b) => a.lo - b.lo);
      for (let i = 1; i < writers.length; i++) if (writers[i].lo < writers[i - 1].hi) return false;
      for (const m of list) {
        let at = m.lo;
        for (const w of writers) {
          if (w.hi <= at) continue;
          if (w.lo > at) break;
          at = w.hi;
          if (at >= m.hi) break;
        }
        if (at < m.hi) return false;
      }
    }
    return true;
  };
  // pieces[i] starts at byte offsets[i] of whole, when dims before `dim` are all 1
  const contiguousPieces = (whole, pieces, dim) => {
    const w = values[whole];
    if (!w || w.type !== 'tensor') return null;
    const d = dim < 0 ? dim + w.shape.length : dim;
    if (!(d >= 0 && d < w.shape.length) || w.shape.slice(0, d).some((n) => n !== 1)) return null;
    const offs = [];
    let at = 0;
    for (const p of pieces) {
      const v = values[p];
      if (!v || v.type !== 'tensor' || v.dtype !== w.dtype) return null;
      offs.push(at);
      at += valueBytes(v);
    }
    return at === valueBytes(w) ? offs : null;
  };

  chain.forEach((op, k) => {
    let ties = null;  // [a, b, delta]: a starts delta bytes after b
    const a = op.args;
    if (op.name === 'aten.cat.default' && a.length === 3 && values[a[0]] && values[a[0]].type === 'tensorlist') {
      const items = values[a[0]].items, y = a[2];
      const offs = contiguousPieces(y, items, values[a[1]].value);
      if (offs) ties = items.map((id, i) => [id, y, offs[i]]);
    } else if (op.name === 'aten.split_with_sizes_copy.default' && a.length === 4 &&
               values[a[3]] && values[a[3]].type === 'tensorlist') {
      const items = values[a[3]].items, x = a[0];
      const offs = contiguousPieces(x, items, values[a[2]].value);
      if (offs) ties = items.map((id, i) => [id, x, offs[i]]);
    } else if (FLAT_COPIES.has(op.name) && a.length === 3 &&
               (op.name !== 'aten.clone.default' || !values[a[1]] || values[a[1]].type === 'null')) {
      const x = a[0], y = a[2];
      if (values[x] && values[y] && values[x].type === 'tensor' && values[y].type === 'tensor' &&
          values[x].dtype === values[y].dtype && valueBytes(values[x]) === valueBytes(values[y])) ties = [[y, x, 0]];
    }
    if (!ties || ties.some(([p, q]) => !movable(p) || !movable(q))) return;
    const saved = [new Map(parent), new Map(offset), new Set(members)];
    elided.add(k);
    let ok = true;
    for (const [p, q, delta] of ties) {
      members.add(p);
      members.add(q);
      if (!tie(p, q, delta)) { ok = false; break; }
    }
    if (!ok || !consistent()) {
      [parent, offset] = saved;
      members.clear();
      saved[2].forEach((id) => members.add(id));
      elided.delete(k);
    }
  });

  // groups start at their lowest member
  const low = new Map(), high = new Map();
  for (const id of members) {
    const [r, d] = find(id);
    low.set(r, Math.min(low.has(r) ? low.get(r) : d, d));
    high.set(r, Math.max(high.has(r) ? high.get(r) : -Infinity, d + valueBytes(values[id])));
  }
  const place = new Map(), groupBytes = new Map();
  for (const id of members) {
    const [r, d] = find(id);
    place.set(id, { root: r, off: d - low.get(r) });
  }
  for (const [r, lo] of low) groupBytes.set(r, high.get(r) - lo);
  return { place, groupBytes, elided };
}

// ------------------------------------------------------------------ operators

const shaders = require('./shaders')({ native, Tensor, DTYPE_BYTESIZE });

/** src/shaders/index.ts:58-60 */
const shaderRegistry = Object.fromEntries
  ? Object.fromEntries(Object.values(shaders).map((s) => [s.name, s]))
  : Object.values(shaders).reduce((o, s) => { o[s.name] = s; return o; }, {});

// ------------------------------------------------------------------ float16 helpers
// Node 12 has no Float16Array: f16 data crosses as Uint16Array bit patterns.

const f32buf = new Float32Array(1);
const u32buf = new Uint32Array(f32buf.buffer);

/** float -> IEEE binary16 bits, round to nearest even. */
function toHalf(f) {
  f32buf[0] = f;
  const x = u32buf[0];
  const sign = (x >>> 16) & 0x8000;
  const ax = x & 0x7fffffff;
  if (ax >= 0x7f800000) return sign | (ax > 0x7f800000 ? 0x7e00 : 0x7c00);
  if (ax >= 0x477ff000) return sign | 0x7c00;
  if (ax < 0x38800000) {
    f32buf[0] = Math.abs(f) * 16777216;
    const s = f32buf[0];
    let m = Math.floor(s);
    const r = s - m;
    if (r > 0.5 || (r === 0.5 && (m & 1))) m += 1;
    return sign | m;
  }
  let h = (((ax >>> 23) - 112) << 10) | ((ax >>> 13) & 0x3ff);
  const rem = ax & 0x1fff;
  if (rem > 0x1000 || (rem === 0x1000 && (h & 1))) h += 1;
  return sign | h;
}

function fromHalf(h) {
  const e = (h >>> 10) & 0x1f;
  const m = h & 0x3ff;
  let v;
  if (e === 0) v = m * Math.pow(2, -24);
  else if (e === 31) v = m ? NaN : Infinity;
  else v = (m + 1024) * Math.pow(2, e - 25);
  return (h & 0x8000) ? -v : v;
}

function toFloat16Array(values) {
  const out = new Uint16Array(values.length);
  for (let i = 0; i < values.length; i++) out[i] = toHalf(values[i]);
  return out;
}

function fromFloat16Array(bits) {
  const u = bits instanceof ArrayBuffer ? new Uint16Array(bits) : bits;
  const out = new Float32Array(u.length);
  for (let i = 0; i < u.length; i++) out[i] = fromHalf(u[i]);
  return out;
}

module.exports = {
  GPUBufferUsage, MAX_NDIM, DTYPE_BYTESIZE, Tensor, WgpuExecutionContext, WgxDevice, WgxBuffer,
  requestDevice, createDevice, resolveArgs, validateProgram, shaders, shaderRegistry, toHalf, fromHalf,
  toFloat16Array, fromFloat16Array, _planViews: planViews,
};
