'use strict';
// createHipRealizerBridge: the HIP realizer behind the reference's
// WebGpuRealizerBridge interface (packages/browsergrad-kernels/src/
// realizer.ts:77-280), for Node hosts.  Method names, argument meaning and
// return types are the reference's; device work runs through bghip.node
// (N-API over libbghip.so).  materialize and the tensor-plan runs return
// Promises that settle when a libuv worker has finished the device call (the
// event loop keeps running meanwhile); the other methods the reference
// declares async return Promises resolved after the native call.
//
//   const { createHipRealizerBridge } = require('./browsergrad_amd/node');
//   const bridge = createHipRealizerBridge({ device: 0 });
//   pyodide.registerJsModule('_bg_webgpu_bridge', bridge);

const path = require('path');

let native = null;
function loadNative() {
  if (native === null) native = require(path.join(__dirname, 'bghip.node'));
  return native;
}

class KernelError extends Error {
  constructor(message) {
    super(message);
    this.name = 'KernelError';
  }
}

// fused_elementwise.ts:83-90 opcodes, as the C ABI numbers them.
const OPCODES = { ADD: 0, MUL: 1, DIV: 2, NEG: 3, EXP: 4, LOG: 5 };

function asBytes(data, name) {
  if (!(data instanceof Uint8Array)) throw new KernelError(`WebGPU bridge: ${name}.data must be Uint8Array bytes`);
  return data;
}

// Native errors named "KernelError" (and rejections of the async bindings)
// become this module's KernelError class.
function asKernelError(e) {
  if (e && e.name === 'KernelError' && !(e instanceof KernelError)) return new KernelError(e.message);
  return e;
}

function wrap(fn) {
  try {
    return fn();
  } catch (e) {
    if (e && e.name === 'KernelError') throw new KernelError(e.message);
    throw e;
  }
}

function createHipRealizerBridge(options = {}) {
  const n = loadNative();
  const ctx = n.ctxCreate(options.device || 0, !!options.profiling);
  const traces = new Map();

  function uploadPlanInputs(plan, inputs) {
    const steps = new Map();
    for (const st of plan.steps || []) steps.set(st.valueId !== undefined ? st.valueId : st.value_id, st);
    const ids = [];
    const handles = [];
    const temps = [];
    try {
      inputs.forEach((input, i) => {
        if (input === null || typeof input !== 'object' || Array.isArray(input)) {
          throw new KernelError(`WebGPU bridge: tensor plan input ${i} must be an object`);
        }
        const id = input.valueId !== undefined ? input.valueId : input.value_id;
        if (!Number.isInteger(id)) throw new KernelError(`WebGPU bridge: tensor plan input ${i}.valueId must be an integer`);
        if (input.handle !== undefined) {
          if (!Number.isInteger(input.handle)) throw new KernelError(`WebGPU bridge: tensor plan input ${i}.handle must be an integer`);
          ids.push(id);
          handles.push(input.handle);
          return;
        }
        const data = asBytes(input.data, `tensor plan input ${i}`);
        const st = steps.get(id);
        const dtype = st ? st.dtype : 'float32';
        const width = dtype === 'float16' || dtype === 'bfloat16' ? 2 : dtype === 'bool' ? 1 : 4;
        if (data.byteLength % width !== 0) {
          throw new KernelError(`WebGPU bridge: tensor plan input ${i}.data byte length must be divisible by ${width}`);
        }
        const h = n.upload(ctx, data, [data.byteLength / width], dtype);
        temps.push(h);
        ids.push(id);
        handles.push(h);
      });
    } catch (e) {
      for (const h of temps) n.release(ctx, h);
      throw e;
    }
    return { ids, handles, temps };
  }

  function rootBytes(plan) {
    const rootId = plan.rootId !== undefined ? plan.rootId : plan.root_id;
    const st = (plan.steps || []).find((s) => (s.valueId !== undefined ? s.valueId : s.value_id) === rootId);
    if (!st) return 0;
    const numel = st.shape.reduce((a, b) => a * b, 1);
    const width = st.dtype === 'float16' || st.dtype === 'bfloat16' ? 2 : st.dtype === 'bool' ? 1 : 4;
    return numel * width;
  }

  // The plan runs on a libuv worker (runTensorPlanAsync); inputs uploaded
  // here are released once it settles.
  async function runPlan(plan, requests, inputs, dtype, resident) {
    const obj = typeof plan === 'string' ? JSON.parse(plan) : plan;
    const text = typeof plan === 'string' ? plan : JSON.stringify(plan);
    const req = requests === null || requests === undefined ? null
      : (typeof requests === 'string' ? requests : JSON.stringify(requests));
    const { ids, handles, temps } = uploadPlanInputs(obj, inputs);
    try {
      return await n.runTensorPlanAsync(ctx, text, req, ids, handles, dtype, resident, rootBytes(obj));
    } catch (e) {
      throw asKernelError(e);
    } finally {
      for (const h of temps) n.release(ctx, h);
    }
  }

  const bridge = {
    upload: (data, shape, dtype) => wrap(() => n.upload(ctx, asBytes(data, 'upload'), shape, dtype)),
    materialize: async (h, _shape, _dtype) => {
      try {
        return await n.materializeAsync(ctx, h);
      } catch (e) {
        throw asKernelError(e);
      }
    },
    release: (h) => wrap(() => n.release(ctx, h)),
    matmul: (a, b, m, k, nn, dtype) => wrap(() => n.matmul(ctx, a, b, m, k, nn, dtype)),
    fused_elementwise: (inputs, ops, shape, dtype) => wrap(() => {
      const flat = [];
      for (const [op, lhs, rhs] of ops) {
        if (!(op in OPCODES)) throw new KernelError(`fused_elementwise: unsupported opcode ${JSON.stringify(op)}`);
        flat.push(OPCODES[op], lhs, rhs === null || rhs === undefined ? lhs : rhs);
      }
      return n.fusedElementwise(ctx, inputs, flat, shape, dtype);
    }),
    cast: (h, srcDtype, dstDtype, shape) => wrap(() => n.cast(ctx, h, srcDtype, dstDtype, shape)),
    flash_attention: async (q, k, v, mask, b, h, sq, sk, d, scale, dtype) =>
      wrap(() => n.flashAttention(ctx, q, k, v, mask, b, h, sq, sk, d, scale, dtype)),
    run_tensor_plan: async (plan, inputs, dtype) => runPlan(plan, null, inputs, dtype, false),
    run_tensor_plan_semantic: async (plan, requests, inputs, dtype) => runPlan(plan, requests, inputs, dtype, false),
    run_tensor_plan_resident: (plan, inputs, dtype) => runPlan(plan, null, inputs, dtype, true),
    run_tensor_plan_resident_semantic: async (plan, requests, inputs, dtype) => {
      const h = await runPlan(plan, requests, inputs, dtype, true);
      traces.set(h, { preparation: typeof requests === 'string' ? JSON.parse(requests) : requests });
      return h;
    },
    semanticTensorPlanExecutionTrace: async (h) => {
      const t = traces.get(h);
      if (!t) throw new KernelError(`WebGPU bridge: handle ${h} has no semantic tensor-plan execution trace`);
      return t;
    },
    aliveHandleCount: () => wrap(() => n.aliveHandles(ctx)),
    resourceSnapshot: () => wrap(() => n.resourceSnapshot(ctx)),
    flushProfiles: async () => wrap(() => ({ ...n.resourceSnapshot(ctx), passProfiles: n.flushProfiles(ctx) })),
    close: () => n.ctxDestroy(ctx),
  };
  // conv1d / conv2d and their backward kernels (realizer.ts:114-238), on the
  // descriptor entry point bg_conv_ex: op 0 forward, 1 input, 2 weight, 3 bias.
  const f32 = (dtype, name) => {
    if (dtype !== 'float32') throw new KernelError(`HIP bridge: ${name} supports float32 only, got ${dtype}`);
  };
  const conv = (op, a, b, bias, nn, cIn, cOut, groups, sp) => wrap(() => n.conv(
    ctx, op, 0, a, b, bias, nn, cIn, cOut, groups, sp.in, sp.out, sp.k, sp.stride, sp.pad, sp.dil,
    sp.in.map(() => 0)));
  const sp1 = (lIn, lOut, k, stride, padding, dilation) =>
    ({ in: [lIn], out: [lOut], k: [k], stride: [stride], pad: [padding], dil: [dilation] });
  const sp2 = (h, w, outH, outW, kh, kw, sh, sw, ph, pw, dh, dw) =>
    ({ in: [h, w], out: [outH, outW], k: [kh, kw], stride: [sh, sw], pad: [ph, pw], dil: [dh, dw] });
  Object.assign(bridge, {
    conv1d: (input, weight, bias, nn, cIn, lIn, cOut, k, stride, padding, dilation, groups, lOut, dtype) => {
      f32(dtype, 'conv1d');
      return conv(0, input, weight, bias, nn, cIn, cOut, groups, sp1(lIn, lOut, k, stride, padding, dilation));
    },
    conv1d_backward_input: (dy, weight, nn, cIn, lIn, cOut, k, stride, padding, dilation, groups, lOut, dtype) => {
      f32(dtype, 'conv1d_backward_input');
      return conv(1, dy, weight, null, nn, cIn, cOut, groups, sp1(lIn, lOut, k, stride, padding, dilation));
    },
    conv1d_backward_weight: (dy, input, nn, cIn, lIn, cOut, k, stride, padding, dilation, groups, lOut, dtype) => {
      f32(dtype, 'conv1d_backward_weight');
      return conv(2, dy, input, null, nn, cIn, cOut, groups, sp1(lIn, lOut, k, stride, padding, dilation));
    },
    conv1d_backward_bias: (dy, nn, cOut, lOut, dtype) => {
      f32(dtype, 'conv1d_backward_bias');
      return conv(3, dy, null, null, nn, cOut, cOut, 1, sp1(lOut, lOut, 1, 1, 0, 1));
    },
    conv2d: (input, weight, bias, nn, cIn, h, w, cOut, kh, kw, sh, sw, ph, pw, dh, dw, groups, outH, outW,
      dtype) => {
      f32(dtype, 'conv2d');
      return conv(0, input, weight, bias, nn, cIn, cOut, groups, sp2(h, w, outH, outW, kh, kw, sh, sw, ph, pw, dh, dw));
    },
    conv2d_backward_input: (dy, weight, nn, cIn, h, w, cOut, kh, kw, sh, sw, ph, pw, dh, dw, groups, outH, outW,
      dtype) => {
      f32(dtype, 'conv2d_backward_input');
      return conv(1, dy, weight, null, nn, cIn, cOut, groups, sp2(h, w, outH, outW, kh, kw, sh, sw, ph, pw, dh, dw));
    },
    conv2d_backward_weight: (dy, input, nn, cIn, h, w, cOut, kh, kw, sh, sw, ph, pw, dh, dw, groups, outH, outW,
      dtype) => {
      f32(dtype, 'conv2d_backward_weight');
      return conv(2, dy, input, null, nn, cIn, cOut, groups, sp2(h, w, outH, outW, kh, kw, sh, sw, ph, pw, dh, dw));
    },
    conv2d_backward_bias: (dy, nn, cOut, outH, outW, dtype) => {
      f32(dtype, 'conv2d_backward_bias');
      return conv(3, dy, null, null, nn, cOut, cOut, 1, sp2(outH, outW, outH, outW, 1, 1, 1, 1, 0, 0, 1, 1));
    },
    run_user_kernel: () => {
      throw new KernelError("HIP bridge: run_user_kernel takes WGSL, which has no HIP meaning");
    },
  });
  return bridge;
}

module.exports = { createHipRealizerBridge, KernelError, version: () => loadNative().version() };
