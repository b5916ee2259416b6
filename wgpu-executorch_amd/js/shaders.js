'use strict';
/**
 * Operator drivers (the Shader objects of src/shaders/<op>/index.ts):
 * `{ name, code, recordIn(ctx, args) }`.  Each recordIn validates its
 * argument tuple with the reference's checks and messages, then appends one
 * native record.  `code` names the MI355X kernels instead of holding WGSL.
 */
module.exports = function makeShaders({ native, DTYPE_BYTESIZE }) {
  const isFloatPair = (t) => t.dtype === 'float32' || t.dtype === 'float16';
  // the GEMM-shaped drivers also take bfloat16 (this backend's addition: the
  // MFMA kernels run it natively); the reference's message stays the same
  const isGemmFloat = (t) => isFloatPair(t) || t.dtype === 'bfloat16';

  function parseHw(name, v, argName) {
    if (v.length === 1) return [v[0], v[0]];
    if (v.length === 2) return [v[0], v[1]];
    throw new Error(`${name}: ${argName} must be 1 or 2 elements`);
  }

  function broadcastable(a, b, out) {
    const n = out.shape.length;
    if (a.shape.length > n || b.shape.length > n) return false;
    for (let k = 0; k < n; k++) {
      const o = out.shape[n - 1 - k];
      const da = k < a.shape.length ? a.shape[a.shape.length - 1 - k] : 1;
      const db = k < b.shape.length ? b.shape[b.shape.length - 1 - k] : 1;
      if ((da !== o && da !== 1) || (db !== o && db !== 1)) return false;
    }
    return true;
  }

  // ---------------------------------------------------------------- mm (src/shaders/mm/index.ts:32-93)
  const mm = {
    name: 'aten.mm.default',
    code: { f32: 'gemm_f32 (vector FMA, LDS-blocked)', f16: 'gemm_mfma (v_mfma_f32_32x32x16_f16)' },
    recordIn(ctx, [in1, in2, out]) {
      const name = 'aten.mm.default';
      if (!isGemmFloat(in1) || in2.dtype !== in1.dtype || out.dtype !== in1.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (in1.shape.length !== 2 || in2.shape.length !== 2 || out.shape.length !== 2) {
        throw new Error(`${name}: Tensors must be 2D matrices`);
      }
      const [m, k1] = in1.shape;
      const [k2, n] = in2.shape;
      const [outM, outN] = out.shape;
      if (k1 !== k2) throw new Error(`${name}: Matrix inner dimensions must match (${k1} !== ${k2})`);
      if (outM !== m || outN !== n) {
        throw new Error(`${name}: Output shape [${outM}, ${outN}] !== expected [${m}, ${n}]`);
      }
      native.recordMm(ctx._h, in1._c(), in2._c(), null, out._c(), 1, 1, 0);
    },
  };

  // ---------------------------------------------------------------- addmm (new: absent from the reference)
  // aten.addmm.default [bias, mat1, mat2, beta?, alpha?, out]: out = beta*bias + alpha*(mat1 @ mat2)
  const addmm = {
    name: 'aten.addmm.default',
    code: { f16: 'gemm_mfma with fused bias epilogue' },
    recordIn(ctx, args) {
      const name = 'aten.addmm.default';
      const [bias, mat1, mat2] = args;
      const out = args[args.length - 1];
      const beta = args.length >= 5 && typeof args[3] === 'number' ? args[3] : 1;
      const alpha = args.length >= 6 && typeof args[4] === 'number' ? args[4] : 1;
      if (!isGemmFloat(mat1) || mat2.dtype !== mat1.dtype || out.dtype !== mat1.dtype || bias.dtype !== mat1.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (mat1.shape.length !== 2 || mat2.shape.length !== 2 || out.shape.length !== 2) {
        throw new Error(`${name}: Tensors must be 2D matrices`);
      }
      const [m, k1] = mat1.shape;
      const [k2, n] = mat2.shape;
      if (k1 !== k2) throw new Error(`${name}: Matrix inner dimensions must match (${k1} !== ${k2})`);
      if (out.shape[0] !== m || out.shape[1] !== n) {
        throw new Error(`${name}: Output shape [${out.shape[0]}, ${out.shape[1]}] !== expected [${m}, ${n}]`);
      }
      native.recordMm(ctx._h, mat1._c(), mat2._c(), bias._c(), out._c(), alpha, beta, 0);
    },
  };

  // Linear layer with the nn.Linear weight layout W[N,K]: [x, weight, bias|undefined, out]
  const linear = {
    name: 'aten.linear.default',
    code: { f16: 'gemm_mfma NT form (k-contiguous weight rows)' },
    recordIn(ctx, [x, weight, bias, out]) {
      const name = 'aten.linear.default';
      if (!isGemmFloat(x) || weight.dtype !== x.dtype || out.dtype !== x.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (x.shape.length !== 2 || weight.shape.length !== 2 || out.shape.length !== 2) {
        throw new Error(`${name}: Tensors must be 2D matrices`);
      }
      if (x.shape[1] !== weight.shape[1]) {
        throw new Error(`${name}: Matrix inner dimensions must match (${x.shape[1]} !== ${weight.shape[1]})`);
      }
      native.recordMm(ctx._h, x._c(), weight._c(), bias === undefined ? null : bias._c(), out._c(), 1, 1, 1);
    },
  };

  // ---------------------------------------------------------------- bmm (src/shaders/bmm/index.ts:27-96)
  const bmm = {
    name: 'aten.bmm.default',
    code: { f32: 'gemm_f32 batched', f16: 'gemm_mfma batched' },
    recordIn(ctx, [a, b, out]) {
      const name = 'aten.bmm.default';
      if (!isGemmFloat(a) || b.dtype !== a.dtype || out.dtype !== a.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (a.shape.length !== 3 || b.shape.length !== 3 || out.shape.length !== 3) {
        throw new Error(`${name}: inputs and output must be 3D`);
      }
      const [batch, m, k] = a.shape;
      const n = b.shape[2];
      if (b.shape[0] !== batch || b.shape[1] !== k) throw new Error(`${name}: batch/K mismatch between a and b`);
      if (out.shape[0] !== batch || out.shape[1] !== m || out.shape[2] !== n) {
        throw new Error(`${name}: output shape [${out.shape}] != [${batch}, ${m}, ${n}]`);
      }
      native.recordBmm(ctx._h, a._c(), b._c(), out._c(), 0);
    },
  };

  // ---------------------------------------------------------------- convolution (src/shaders/convolution/index.ts:58-310)
  // activation: 0 none, 1 SiLU folded into the epilogue (recordProgram's
  // conv -> sigmoid -> mul fusion; the reference operators never pass it)
  // residual: {tensor, convScale, residualScale} adds an output-shaped tensor
  // after the epilogue (recordProgram's folding of a following add)
  function recordConv(name, ctx, inTensor, weight, bias, stride, padding, dilation, transposed, outputPadding,
    groups, outTensor, clampMin, clampMax, activation, residual) {
    if (!isGemmFloat(inTensor) || weight.dtype !== inTensor.dtype || outTensor.dtype !== inTensor.dtype) {
      throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
    }
    if (bias !== undefined && bias.dtype !== inTensor.dtype) {
      throw new Error(`${name}: bias dtype must match input dtype`);
    }
    if (inTensor.shape.length !== 4 || weight.shape.length !== 4 || outTensor.shape.length !== 4) {
      throw new Error(`${name}: expected 4D tensors for input, weight, and output`);
    }
    const [sH, sW] = parseHw(name, stride, 'stride');
    const [pH, pW] = parseHw(name, padding, 'padding');
    const [dH, dW] = parseHw(name, dilation, 'dilation');
    const [opH, opW] = parseHw(name, outputPadding, 'output_padding');
    const [, ic, ih, iw] = inTensor.shape;
    const kh = weight.shape[2];
    const kw = weight.shape[3];
    if (transposed) {
      if (weight.shape[0] !== ic) throw new Error(`${name}: weight dim0 !== IC (${weight.shape[0]} != ${ic})`);
      if (opH >= sH || opW >= sW) throw new Error(`${name}: output_padding >= stride`);
      const eoh = (ih - 1) * sH - 2 * pH + dH * (kh - 1) + opH + 1;
      const eow = (iw - 1) * sW - 2 * pW + dW * (kw - 1) + opW + 1;
      if (outTensor.shape[2] !== eoh || outTensor.shape[3] !== eow) {
        throw new Error(`${name}: expected output spatial [${eoh}, ${eow}]`);
      }
    } else {
      if (outputPadding.some((v) => v !== 0)) {
        throw new Error(`${name}: non-zero output_padding unsupported for non-transposed conv`);
      }
      if (weight.shape[1] !== ic / groups) {
        throw new Error(`${name}: weight in-ch (${weight.shape[1]}) != IC/groups (${ic / groups})`);
      }
      const ohNum = ih + 2 * pH - dH * (kh - 1) - 1;
      const owNum = iw + 2 * pW - dW * (kw - 1) - 1;
      if (ohNum < 0 || owNum < 0) throw new Error(`${name}: invalid geometry (kernel larger than input)`);
      const eoh = Math.floor(ohNum / sH) + 1;
      const eow = Math.floor(owNum / sW) + 1;
      if (outTensor.shape[2] !== eoh || outTensor.shape[3] !== eow) {
        throw new Error(`${name}: expected output spatial [${eoh}, ${eow}]`);
      }
    }
    // The reference's generic im2col GEMM variant (dense, not 1x1, K not a
    // multiple of 4 or fewer than 64 output pixels, or OC < 8) launches one
    // workgroup per 32 x 32 tile and refuses grids past 65535 in either
    // direction (src/shaders/convolution/index.ts:168-205, 278-286); the
    // MI355X kernels have no such limit, but the drop-in keeps the refusal.
    const [b] = inTensor.shape;
    const oc = outTensor.shape[1];
    const nPix = b * outTensor.shape[2] * outTensor.shape[3];
    if (name === 'aten.convolution.default' && !transposed && groups === 1) {
      const is1x1 = kh === 1 && kw === 1 && sH === 1 && sW === 1 && pH === 0 && pW === 0 && dH === 1 && dW === 1;
      const is1x1Vec4 = is1x1 && ic % 4 === 0 && (outTensor.shape[2] * outTensor.shape[3]) % 4 === 0 && oc % 4 === 0;
      const is1x1Tiled = is1x1Vec4 && b === 1 && outTensor.shape[2] * outTensor.shape[3] >= 64 && ic >= 16;
      const isDenseTiled = oc >= 8 && nPix >= 64 && (ic * kh * kw) % 4 === 0;
      const isF16 = inTensor.dtype === 'float16';
      const isDepthwise = oc === 1 && ic === 1 && kh * kw <= 49 && b <= 65535;  // groups === oc === ic
      const generic = !isDepthwise && !is1x1Tiled && !isDenseTiled && !(is1x1 && !isF16);
      if (generic && (Math.ceil(nPix / 32) > 65535 || Math.ceil(oc / 32) > 65535)) {
        throw new Error(`${name}: GEMM tile grid exceeds dispatch limit`);
      }
    }
    const hasClamp = clampMin !== undefined || clampMax !== undefined;
    native.recordConv2d(ctx._h, inTensor._c(), weight._c(), bias === undefined ? null : bias._c(), {
      stride: [sH, sW], padding: [pH, pW], dilation: [dH, dW], outputPadding: [opH, opW],
      transposed: transposed ? 1 : 0, groups, hasClamp: hasClamp ? 1 : 0,
      clampMin: clampMin === undefined ? -Infinity : clampMin,
      clampMax: clampMax === undefined ? Infinity : clampMax,
      activation: activation || 0,
      residual: residual ? residual.tensor._c() : null,
      convScale: residual ? residual.convScale : 1,
      residualScale: residual ? residual.residualScale : 0,
    }, outTensor._c());
  }

  /** aten.convolution.default followed by SiLU (x * sigmoid(x)) in one launch. */
  const convolutionSilu = {
    name: 'wgx.convolution_silu',
    code: { all: 'the convolution kernels with the SiLU epilogue enabled' },
    recordIn(ctx, args) {
      const [inTensor, weight, bias, stride, padding, dilation, transposed, outputPadding, groups, outTensor] = args;
      recordConv('aten.convolution.default', ctx, inTensor, weight, bias, stride, padding, dilation, transposed,
        outputPadding, groups, outTensor, undefined, undefined, 1);
    },
  };

  /**
   * aten.convolution.default, SiLU, then aten.add.Tensor with an
   * output-shaped tensor, in one launch (depthwise convolutions and the
   * dense 3x3 ones the LDS-patch kernel takes; the native layer refuses the
   * rest): out = convScale * silu(conv) + residualScale * residual.
   */
  const convolutionSiluAdd = {
    name: 'wgx.convolution_silu_add',
    code: { all: 'the depthwise and LDS-patch convolution kernels with the SiLU and residual epilogue' },
    recordIn(ctx, args) {
      const [inTensor, weight, bias, stride, padding, dilation, transposed, outputPadding, groups, residual,
        convScale, residualScale, outTensor] = args;
      if (residual.dtype !== outTensor.dtype || residual.shape.length !== outTensor.shape.length ||
          residual.shape.some((d, i) => d !== outTensor.shape[i])) {
        throw new Error('wgx.convolution_silu_add: residual must match the output dtype and shape');
      }
      recordConv('aten.convolution.default', ctx, inTensor, weight, bias, stride, padding, dilation, transposed,
        outputPadding, groups, outTensor, undefined, undefined, 1, { tensor: residual, convScale, residualScale });
    },
  };

  const convolution = {
    name: 'aten.convolution.default',
    code: {
      gemm: 'gemm_mfma / gemm_f32 implicit-im2col (B_CONV) and 1x1 (B_KN)',
      depthwise: 'depthwise (LDS-banded stencil)', fallback: 'conv_grouped_direct / conv_transpose_direct',
    },
    recordIn(ctx, args) {
      const [inTensor, weight, bias, stride, padding, dilation, transposed, outputPadding, groups, outTensor] = args;
      recordConv('aten.convolution.default', ctx, inTensor, weight, bias, stride, padding, dilation, transposed,
        outputPadding, groups, outTensor);
    },
  };

  // src/shaders/conv-with-clamp/index.ts:60-319: bias, then clamp, then narrow
  const convWithClamp = {
    name: 'et_vk.conv_with_clamp.default',
    code: { all: 'the convolution kernels with the clamp epilogue enabled' },
    recordIn(ctx, args) {
      const [inTensor, weight, bias, stride, padding, dilation, transposed, outputPadding, groups, outMin, outMax,
        outTensor] = args;
      recordConv('et_vk.conv_with_clamp.default', ctx, inTensor, weight, bias, stride, padding, dilation, transposed,
        outputPadding, groups, outTensor, outMin === undefined ? undefined : outMin,
        outMax === undefined ? undefined : outMax);
    },
  };

  // ---------------------------------------------------------------- elementwise
  function binary(name, isAdd, sign) {
    return {
      name,
      code: { all: 'binary broadcast kernel' },
      recordIn(ctx, args) {
        const [in1, in2] = args;
        const alpha = args.length === 4 ? args[2] : 1;
        const out = args[args.length - 1];
        if (!isFloatPair(in1) || in2.dtype !== in1.dtype || out.dtype !== in1.dtype) {
          throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
        }
        if (!broadcastable(in1, in2, out)) throw new Error(`${name}: Input shapes are not broadcastable to output shape`);
        if (isAdd) native.recordAdd(ctx._h, in1._c(), in2._c(), alpha, sign < 0 ? 1 : 0, out._c());
        else native.recordMul(ctx._h, in1._c(), in2._c(), out._c());
      },
    };
  }
  const add = binary('aten.add.Tensor', true, 1);
  const sub = binary('aten.sub.Tensor', true, -1);
  const mul = {
    name: 'aten.mul.Tensor',
    code: { all: 'binary broadcast kernel' },
    recordIn(ctx, [in1, in2, out]) {
      const name = 'aten.mul.Tensor';
      if (!isFloatPair(in1) || in2.dtype !== in1.dtype || out.dtype !== in1.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (!broadcastable(in1, in2, out)) throw new Error(`${name}: Input shapes are not broadcastable to output shape`);
      native.recordMul(ctx._h, in1._c(), in2._c(), out._c());
    },
  };

  function unary(name, op) {
    return {
      name,
      code: { all: 'unary kernel' },
      recordIn(ctx, [inTensor, outTensor]) {
        if (!isFloatPair(inTensor) || outTensor.dtype !== inTensor.dtype) {
          throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
        }
        if (inTensor.numel !== outTensor.numel) throw new Error(`${name}: input numel != output numel`);
        native.recordUnary(ctx._h, op, inTensor._c(), outTensor._c());
      },
    };
  }
  const sigmoid = unary('aten.sigmoid.default', 0);
  const relu = unary('aten.relu.default', 1);
  const hardswish = unary('aten.hardswish.default', 2);

  // ---------------------------------------------------------------- data movement
  const cat = {
    name: 'aten.cat.default',
    code: { all: 'slab copy kernel per input' },
    recordIn(ctx, [tensors, dim, out]) {
      const name = 'aten.cat.default';
      if (tensors.length === 0) throw new Error(`${name}: empty input list`);
      const rank = out.shape.length;
      const d = dim < 0 ? dim + rank : dim;
      if (d < 0 || d >= rank) throw new Error(`${name}: dim out of range`);
      let total = 0;
      for (const t of tensors) {
        if (t.dtype !== out.dtype || !isFloatPair(t)) throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
        if (t.shape.length !== rank) throw new Error(`${name}: input rank != output rank`);
        for (let k = 0; k < rank; k++) {
          if (k !== d && t.shape[k] !== out.shape[k]) throw new Error(`${name}: non-concat dim ${k} size mismatch`);
        }
        total += t.shape[d];
      }
      if (total !== out.shape[d]) throw new Error(`${name}: concat dim sizes do not sum to output`);
      native.recordCat(ctx._h, tensors.map((t) => t._c()), d, out._c());
    },
  };

  const splitWithSizesCopy = {
    name: 'aten.split_with_sizes_copy.default',
    code: { all: 'slab gather kernel per output' },
    recordIn(ctx, [inTensor, splitSizes, dim, outs]) {
      const name = 'aten.split_with_sizes_copy.default';
      const rank = inTensor.shape.length;
      const d = dim < 0 ? dim + rank : dim;
      if (d < 0 || d >= rank) throw new Error(`${name}: dim out of range`);
      if (outs.length !== splitSizes.length) throw new Error(`${name}: outputs (${outs.length}) != sizes (${splitSizes.length})`);
      if (splitSizes.some((s) => s < 0)) throw new Error(`${name}: negative split size`);
      if (splitSizes.reduce((a, b) => a + b, 0) !== inTensor.shape[d]) {
        throw new Error(`${name}: sizes must sum to the split dim extent`);
      }
      outs.forEach((t, i) => {
        if (t.dtype !== inTensor.dtype || !isFloatPair(t)) throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
        if (t.shape[d] !== splitSizes[i]) throw new Error(`${name}: output ${i} dim ${d} != split size`);
      });
      native.recordSplit(ctx._h, inTensor._c(), d, outs.map((t) => t._c()));
    },
  };

  const upsampleNearest2d = {
    name: 'aten.upsample_nearest2d.vec',
    code: { all: 'nearest upsample kernel' },
    recordIn(ctx, [inTensor, , , outTensor]) {
      const name = 'aten.upsample_nearest2d.vec';
      if (!isFloatPair(inTensor) || outTensor.dtype !== inTensor.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (inTensor.shape.length !== 4 || outTensor.shape.length !== 4) throw new Error(`${name}: input and output must be 4D NCHW`);
      if (inTensor.shape[0] !== outTensor.shape[0] || inTensor.shape[1] !== outTensor.shape[1]) {
        throw new Error(`${name}: output batch/channels must match input`);
      }
      if (outTensor.shape[2] < inTensor.shape[2] || outTensor.shape[3] < inTensor.shape[3]) {
        throw new Error(`${name}: output spatial dims must be >= input spatial dims`);
      }
      native.recordUpsampleNearest2d(ctx._h, inTensor._c(), outTensor._c());
    },
  };

  // src/shaders/max-pool-2d/index.ts:41-106: values and int32 indices
  const maxPool2d = {
    name: 'aten.max_pool2d_with_indices.default',
    code: { all: 'max-pool kernel (values and indices); chained same-size pools fold into one launch' },
    recordIn(ctx, [inTensor, kernelSize, stride, padding, dilation, ceilMode, outs]) {
      const name = 'aten.max_pool2d_with_indices.default';
      if (outs.length !== 2) throw new Error(`${name}: expected 2 outputs [values, indices], got ${outs.length}`);
      const [vals, idx] = outs;
      if (!isFloatPair(inTensor) || vals.dtype !== inTensor.dtype) {
        throw new Error(`${name}: values tensors must have matching float32 or float16 dtype`);
      }
      if (idx.dtype !== 'int32') throw new Error(`${name}: indices output must be int32`);
      if (inTensor.shape.length !== 4) throw new Error(`${name}: input must be 4D NCHW`);
      const [b, c, ih, iw] = inTensor.shape;
      const [kH, kW] = parseHw(name, kernelSize, 'kernel_size');
      const [sH, sW] = parseHw(name, stride, 'stride');
      const [pH, pW] = parseHw(name, padding, 'padding');
      const [dH, dW] = parseHw(name, dilation, 'dilation');
      const ohNum = ih + 2 * pH - (dH * (kH - 1) + 1);
      const owNum = iw + 2 * pW - (dW * (kW - 1) + 1);
      const oh = Math.max(0, (ceilMode ? Math.ceil(ohNum / sH) : Math.floor(ohNum / sH)) + 1);
      const ow = Math.max(0, (ceilMode ? Math.ceil(owNum / sW) : Math.floor(owNum / sW)) + 1);
      const want = [b, c, oh, ow];
      const same = (t) => t.shape.length === 4 && t.shape.every((v, i) => v === want[i]);
      if (!same(vals)) throw new Error(`${name}: values output shape ${vals.shape} != [${want.join(', ')}]`);
      if (!same(idx)) throw new Error(`${name}: indices output shape ${idx.shape} != [${want.join(', ')}]`);
      native.recordMaxPool2d(ctx._h, inTensor._c(), [kH, kW], [sH, sW], [pH, pW], [dH, dW], ceilMode ? 1 : 0,
        vals._c(), idx._c());
    },
  };

  // src/shaders/permute/index.ts:33-99
  const permuteCopy = {
    name: 'aten.permute_copy.default',
    code: { transpose: 'permute_transpose (64x64 LDS tiles, last two dims swapped)', other: 'permute_gather' },
    recordIn(ctx, [inTensor, dims, outTensor]) {
      const name = 'aten.permute_copy.default';
      if (!isFloatPair(inTensor) || outTensor.dtype !== inTensor.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      const rank = inTensor.shape.length;
      if (outTensor.shape.length !== rank) throw new Error(`${name}: output rank != input rank`);
      if (dims.length !== rank) throw new Error(`${name}: dims count (${dims.length}) != input rank (${rank})`);
      const perm = [];
      const seen = new Set();
      for (let d = 0; d < rank; d++) {
        let p = dims[d];
        if (p < 0) p += rank;
        if (p < 0 || p >= rank || seen.has(p)) throw new Error(`${name}: invalid permute dims ${dims}`);
        seen.add(p);
        perm.push(p);
      }
      for (let d = 0; d < rank; d++) {
        if (outTensor.shape[d] !== inTensor.shape[perm[d]]) {
          throw new Error(`${name}: output shape does not match permuted input shape`);
        }
      }
      native.recordPermute(ctx._h, inTensor._c(), perm, outTensor._c());
    },
  };

  // src/shaders/softmax/index.ts:62-125
  const softmax = {
    name: 'aten._softmax.default',
    code: { rows: 'softmax_rows (a wave per contiguous row)', other: 'softmax_strided' },
    recordIn(ctx, [inTensor, dim, , outTensor]) {
      const name = 'aten._softmax.default';
      if (!isFloatPair(inTensor) || outTensor.dtype !== inTensor.dtype) {
        throw new Error(`${name}: Tensors must have matching float32 or float16 dtype`);
      }
      if (inTensor.shape.length === 0) throw new Error(`${name}: scalar input unsupported`);
      if (inTensor.numel !== outTensor.numel) throw new Error(`${name}: input/output numel mismatch`);
      const ndim = inTensor.shape.length;
      const d = dim < 0 ? dim + ndim : dim;
      if (d < 0 || d >= ndim) throw new Error(`${name}: dim out of range`);
      native.recordSoftmax(ctx._h, inTensor._c(), d, outTensor._c());
    },
  };

  function flatCopy(name) {
    return {
      name,
      code: { all: 'device copy (elided when in and out alias)' },
      recordIn(ctx, args) {
        const src = args[0];
        const out = args[args.length - 1];
        if (src.byteLength !== out.byteLength) throw new Error(`${name}: input and output sizes differ`);
        native.recordCopy(ctx._h, out.buffer.ptr, src.buffer.ptr, src.byteLength);
      },
    };
  }

  return {
    add, sub, mul, sigmoid, relu, hardswish,
    mm, addmm, linear, bmm,
    convolution, convWithClamp, convolutionSilu, convolutionSiluAdd, maxPool2d,
    upsampleNearest2d, permuteCopy, softmax,
    cat, splitWithSizesCopy,
    viewCopy: flatCopy('aten.view_copy.default'),
    clone: flatCopy('aten.clone.default'),
    squeezeCopy: flatCopy('aten.squeeze_copy.dims'),
    unsqueezeCopy: flatCopy('aten.unsqueeze_copy.default'),
    prepack: flatCopy('et_vk.prepack.default'),
  };
};
