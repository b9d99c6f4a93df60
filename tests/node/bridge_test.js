'use strict';
// createHipRealizerBridge on the GPU, driven by tests/test_node_bridge.py.
// Known answers are the reference's own:
//   matmul [[1,2],[3,4]]·[[5,6],[7,8]] = [19,22,43,50]   webgpu_real.test.ts:1558-1589
//   fused exp(a+b)/a (closed form per element)           webgpu_real.test.ts:1431-1472
//   attention CS336 non-causal rows                      flash_attention_oracle.test.ts:16-52
//   conv1d / conv2d and conv1d backward known answers    webgpu_real.test.ts:943-1203
//   residency: upload/release/alive bookkeeping          realizer.ts:906-943
const assert = require('assert');
const path = require('path');
const { createHipRealizerBridge, KernelError } = require(path.join(__dirname, '..', '..', 'browsergrad_amd', 'node'));

const f32 = (xs) => new Uint8Array(new Float32Array(xs).buffer);
const fromBytes = (u8) => new Float32Array(u8.buffer, u8.byteOffset, u8.byteLength / 4);
const close = (got, want, tol, what) => {
  assert.strictEqual(got.length, want.length, what);
  for (let i = 0; i < want.length; i++) {
    const d = Math.abs(got[i] - want[i]);
    assert.ok(d <= tol || d <= tol * Math.abs(want[i]), `${what}[${i}]: ${got[i]} vs ${want[i]}`);
  }
};

async function main() {
  const br = createHipRealizerBridge({ device: 0, profiling: true });
  const alive0 = br.aliveHandleCount();

  console.log('[node] matmul known answer');
  const a = br.upload(f32([1, 2, 3, 4]), [2, 2], 'float32');
  const b = br.upload(f32([5, 6, 7, 8]), [2, 2], 'float32');
  const c = br.matmul(a, b, 2, 2, 2, 'float32');
  close(fromBytes(await br.materialize(c, [2, 2], 'float32')), [19, 22, 43, 50], 0, 'matmul');

  console.log('[node] fused exp(a+b)/a');
  const xa = [0.5, 1.0, -2.0, 3.0];
  const xb = [0.25, -1.0, 0.5, 0.125];
  const ha = br.upload(f32(xa), [4], 'float32');
  const hb = br.upload(f32(xb), [4], 'float32');
  const hf = br.fused_elementwise([ha, hb], [['ADD', -1, -2], ['EXP', 0, null], ['DIV', 1, -1]], [4], 'float32');
  close(fromBytes(await br.materialize(hf, [4], 'float32')), xa.map((x, i) => Math.exp(x + xb[i]) / x), 1e-5, 'fused');

  console.log('[node] attention CS336');
  const q = br.upload(f32([1, 0, 0, 1]), [1, 1, 2, 2], 'float32');
  const k = br.upload(f32([1, 0, 0, 1]), [1, 1, 2, 2], 'float32');
  const v = br.upload(f32([10, 20, 30, 40]), [1, 1, 2, 2], 'float32');
  const o = await br.flash_attention(q, k, v, null, 1, 1, 2, 2, 2, 1.0, 'float32');
  close(fromBytes(await br.materialize(o, [1, 1, 2, 2], 'float32')),
        [15.378828, 25.378828, 24.621172, 34.621172], 1e-4, 'attention');

  console.log('[node] cast f32 -> f16 -> f32');
  const h16 = br.cast(ha, 'float32', 'float16', [4]);
  const back = br.cast(h16, 'float16', 'float32', [4]);
  close(fromBytes(await br.materialize(back, [4], 'float32')), xa, 0, 'cast');

  console.log('[node] run_tensor_plan (semantic) and resident');
  const plan = {
    steps: [
      { step: 0, value_id: 0, op: 'BUFFER', input_ids: [], shape: [2, 3], dtype: 'float32', arg: 'x' },
      { step: 1, value_id: 1, op: 'LOAD', input_ids: [0], shape: [2, 3], dtype: 'float32', arg: null },
      { step: 2, value_id: 2, op: 'PERMUTE', input_ids: [1], shape: [3, 2], dtype: 'float32', arg: null },
      { step: 3, value_id: 3, op: 'EXP', input_ids: [2], shape: [3, 2], dtype: 'float32', arg: null },
    ],
    buffers: [],
    root_id: 3, materialization_boundary: 'root', peak_live_bytes: 0, has_custom_ops: false,
  };
  const requests = {
    schema: 'browsergrad.jit.tensor-plan-semantic-requests', version: { major: 1, minor: 0 },
    requests: [{ kind: 'dense-permutation-view-copy', valueId: 2, inputShape: ['2', '3'], axes: [1, 0], dtype: 'f32' }],
  };
  const x = [0, 1, 2, 3, 4, 5];
  const want = [0, 3, 1, 4, 2, 5].map((i) => Math.exp(x[i]));
  const bytes = await br.run_tensor_plan_semantic(plan, requests, [{ valueId: 0, data: f32(x) }], 'float32');
  close(fromBytes(bytes), want, 1e-6, 'plan');
  const root = await br.run_tensor_plan_resident_semantic(plan, requests, [{ valueId: 0, data: f32(x) }], 'float32');
  close(fromBytes(await br.materialize(root, [3, 2], 'float32')), want, 1e-6, 'resident plan');
  assert.strictEqual((await br.semanticTensorPlanExecutionTrace(root)).preparation.requests[0].valueId, 2);

  console.log('[node] conv1d / conv2d known answers');
  // webgpu_real.test.ts:943-1203
  const cx = br.upload(f32([1, 2, 3, 4]), [1, 1, 4], 'float32');
  const cw = br.upload(f32([2, -1]), [1, 1, 2], 'float32');
  const cb = br.upload(f32([0.5]), [1], 'float32');
  const cy = br.conv1d(cx, cw, cb, 1, 1, 4, 1, 2, 1, 0, 1, 1, 3, 'float32');
  close(fromBytes(await br.materialize(cy, [1, 1, 3], 'float32')), [0.5, 1.5, 2.5], 0, 'conv1d');
  const cdy = br.upload(f32([10, 20, 30]), [1, 1, 3], 'float32');
  const cdx = br.conv1d_backward_input(cdy, cw, 1, 1, 4, 1, 2, 1, 0, 1, 1, 3, 'float32');
  close(fromBytes(await br.materialize(cdx, [1, 1, 4], 'float32')), [20, 30, 40, -30], 0, 'conv1d dx');
  const cdw = br.conv1d_backward_weight(cdy, cx, 1, 1, 4, 1, 2, 1, 0, 1, 1, 3, 'float32');
  close(fromBytes(await br.materialize(cdw, [1, 1, 2], 'float32')), [140, 200], 0, 'conv1d dw');
  const cdb = br.conv1d_backward_bias(cdy, 1, 1, 3, 'float32');
  close(fromBytes(await br.materialize(cdb, [1], 'float32')), [60], 0, 'conv1d db');
  const x2 = br.upload(f32([1, 2, 3, 4, 5, 6, 7, 8, 9]), [1, 1, 3, 3], 'float32');
  const w2 = br.upload(f32([1, 0, 0, -1]), [1, 1, 2, 2], 'float32');
  const y2 = br.conv2d(x2, w2, cb, 1, 1, 3, 3, 1, 2, 2, 1, 1, 0, 0, 1, 1, 1, 2, 2, 'float32');
  close(fromBytes(await br.materialize(y2, [1, 1, 2, 2], 'float32')), [-3.5, -3.5, -3.5, -3.5], 0, 'conv2d');
  for (const h of [cx, cw, cb, cy, cdy, cdx, cdw, cdb, x2, w2, y2]) br.release(h);

  console.log('[node] errors are KernelError');
  assert.throws(() => br.matmul(a, 999999, 2, 2, 2, 'float32'), (e) => e.name === 'KernelError');
  await assert.rejects(br.run_tensor_plan_semantic(plan, { ...requests, requests: [] },
                                                   [{ valueId: 0, data: f32(x) }], 'float32'),
                       (e) => e instanceof KernelError && /expected exactly 1 request/.test(e.message));
  assert.throws(() => br.conv2d(), (e) => e.name === 'KernelError');
  assert.throws(() => br.run_user_kernel(), (e) => e.name === 'KernelError');

  console.log('[node] read-backs settle from libuv workers');
  const pending = br.materialize(c, [2, 2], 'float32');
  assert.ok(pending instanceof Promise);
  let ticked = false;
  const tick = new Promise((resolve) => setImmediate(() => { ticked = true; resolve(); }));
  const [m1, m2] = await Promise.all([pending, br.materialize(hf, [4], 'float32'), tick]);
  assert.ok(ticked);
  close(fromBytes(m1), [19, 22, 43, 50], 0, 'async materialize');
  close(fromBytes(m2), xa.map((x, i) => Math.exp(x + xb[i]) / x), 1e-5, 'async materialize 2');
  const gone = br.upload(f32([1, 2]), [2], 'float32');
  br.release(gone);
  await assert.rejects(br.materialize(gone, [2], 'float32'), (e) => e instanceof KernelError);
  const planRuns = await Promise.all([0, 1, 2].map(() => br.run_tensor_plan_semantic(
    plan, requests, [{ valueId: 0, data: f32(x) }], 'float32')));
  for (const pr of planRuns) close(fromBytes(pr), want, 1e-6, 'concurrent plan runs');

  console.log('[node] residency bookkeeping');
  for (const h of [a, b, c, ha, hb, hf, q, k, v, o, h16, back, root]) br.release(h);
  br.release(a);  // idempotent
  assert.strictEqual(br.aliveHandleCount(), alive0);
  const snap = await br.flushProfiles();
  assert.ok(snap.passProfiles.length > 0 && snap.timingMode === 'hip-event');
  br.close();
  console.log('[node] ok');
}

main().catch((e) => {
  console.error('[node] FAILED', e && e.stack ? e.stack : e);
  process.exit(1);
});
