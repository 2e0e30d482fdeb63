// End-to-end check of the Node-API binding on a GPU: allocate through the
// addon, upload, run a GEMM, a cross-entropy forward/backward and one Adam
// step, read back with d2hAsync, and compare with float64 JavaScript
// restatements of the same arithmetic.  Prints one JSON line; exits 1 on a
// mismatch.
'use strict';
const path = require('path');
const hip = require(path.join(__dirname, 'torchjs_hip.node'));

function lcg(seed) {
  let s = seed >>> 0;
  return () => {
    s = (Math.imul(s, 1664525) + 1013904223) >>> 0;
    return s / 4294967296 - 0.5;
  };
}

function upload(arr) {
  const buf = hip.malloc(arr.byteLength);
  hip.h2d(buf.ptr, arr);
  return buf;
}

async function main() {
  hip.init(0);
  const info = hip.deviceInfo();
  const rnd = lcg(7);
  const out = { device: info.arch, version: hip.version };
  let ok = true;

  // GEMM C[M,N] = A[M,K] B[K,N] + bias[N]
  const M = 67, N = 45, K = 33;
  const A = Float32Array.from({ length: M * K }, rnd);
  const Bm = Float32Array.from({ length: K * N }, rnd);
  const bias = Float32Array.from({ length: N }, rnd);
  const dA = upload(A), dB = upload(Bm), dBias = upload(bias);
  const dC = hip.malloc(M * N * 4);
  hip.gemm(0, 0, M, N, K, 1.0, dA.ptr, K, 0, dB.ptr, N, 0, 0.0, dC.ptr, N, 0, 1, dBias.ptr, 1);
  const C = await hip.d2hAsync(dC.ptr, new Float32Array(M * N));
  let gemmErr = 0;
  for (let i = 0; i < M; ++i) {
    for (let j = 0; j < N; ++j) {
      let s = bias[j];
      for (let k = 0; k < K; ++k) s += A[i * K + k] * Bm[k * N + j];
      gemmErr = Math.max(gemmErr, Math.abs(C[i * N + j] - s));
    }
  }
  out.gemm_max_abs_err = gemmErr;
  ok = ok && gemmErr < 1e-5;

  // cross_entropy (mean) forward + backward
  const R = 9, V = 101;
  const logits = Float32Array.from({ length: R * V }, () => 4 * rnd());
  const tg = Int32Array.from({ length: R }, (_, i) => (i * 37) % V);
  tg[3] = -100;  // ignore_index
  const dL = upload(logits), dT = upload(tg);
  const dLse = hip.malloc(R * 4), dRows = hip.malloc(R * 4), dLoss = hip.malloc(4);
  hip.crossEntropyForward(dL.ptr, V, dT.ptr, R, V, -100, null, 0, dLse.ptr, dRows.ptr, 1,
                          dLoss.ptr);
  const one = upload(Float32Array.of(1));
  const dG = hip.malloc(R * V * 4);
  hip.crossEntropyBackward(dL.ptr, V, dT.ptr, null, 0, dLse.ptr, one.ptr, R, V, -100, 1, dG.ptr,
                           V, 0);
  const loss = (await hip.d2hAsync(dLoss.ptr, new Float32Array(1)))[0];
  const grad = await hip.d2hAsync(dG.ptr, new Float32Array(R * V));
  let ref = 0, valid = 0, gErr = 0;
  const lse = [];
  for (let r = 0; r < R; ++r) {
    let mx = -Infinity;
    for (let c = 0; c < V; ++c) mx = Math.max(mx, logits[r * V + c]);
    let s = 0;
    for (let c = 0; c < V; ++c) s += Math.exp(logits[r * V + c] - mx);
    lse.push(mx + Math.log(s));
    if (tg[r] !== -100) { ref += lse[r] - logits[r * V + tg[r]]; valid += 1; }
  }
  ref /= valid;
  for (let r = 0; r < R; ++r) {
    for (let c = 0; c < V; ++c) {
      let g = 0;
      if (tg[r] !== -100) g = (Math.exp(logits[r * V + c] - lse[r]) - (c === tg[r] ? 1 : 0)) / valid;
      gErr = Math.max(gErr, Math.abs(grad[r * V + c] - g));
    }
  }
  out.ce_loss = loss;
  out.ce_loss_err = Math.abs(loss - ref);
  out.ce_grad_max_abs_err = gErr;
  ok = ok && out.ce_loss_err < 1e-5 * Math.max(1, Math.abs(ref)) && gErr < 1e-6;

  // one Adam step (coupled weight decay), step 1
  const P = 1000;
  const p = Float32Array.from({ length: P }, rnd);
  const g = Float32Array.from({ length: P }, rnd);
  const dp = upload(p), dg = upload(g);
  const dm = upload(new Float32Array(P)), dv = upload(new Float32Array(P));
  const lr = 1e-3, b1 = 0.9, b2 = 0.999, eps = 1e-8, wd = 0.01;
  hip.adamStep([dp.ptr], [dg.ptr], [dm.ptr], [dv.ptr], [P], [1], lr, b1, b2, eps, wd, 0);
  const p1 = await hip.d2hAsync(dp.ptr, new Float32Array(P));
  let aErr = 0;
  for (let i = 0; i < P; ++i) {
    const gg = g[i] + p[i] * wd;
    const m = (1 - b1) * gg, v = (1 - b2) * gg * gg;
    const upd = lr / (1 - b1) * m / (Math.sqrt(v / (1 - b2)) + eps);
    aErr = Math.max(aErr, Math.abs(p1[i] - (p[i] - upd)));
  }
  out.adam_max_abs_err = aErr;
  ok = ok && aErr < 1e-6;

  // conv2d forward (NCHW, stride 2, pad 1, bias) against a direct loop
  const cn = 2, cc = 3, ch = 9, cw = 7, coc = 4, k = 3, cs = 2, cp = 1;
  const coh = Math.floor((ch + 2 * cp - k) / cs) + 1, cow = Math.floor((cw + 2 * cp - k) / cs) + 1;
  const cx = Float32Array.from({ length: cn * cc * ch * cw }, rnd);
  const cwt = Float32Array.from({ length: coc * cc * k * k }, rnd);
  const cb = Float32Array.from({ length: coc }, rnd);
  const dcx = upload(cx), dcw = upload(cwt), dcb = upload(cb);
  const dcy = hip.malloc(cn * coc * coh * cow * 4);
  hip.conv2dForward([cn, cc, ch, cw, coc, k, k, cs, cs, cp, cp, 1, 1, 1, coh, cow], dcx.ptr,
                    dcw.ptr, dcb.ptr, dcy.ptr);
  const cy = await hip.d2hAsync(dcy.ptr, new Float32Array(cn * coc * coh * cow));
  let cErr = 0;
  for (let n = 0; n < cn; ++n)
    for (let o = 0; o < coc; ++o)
      for (let y = 0; y < coh; ++y)
        for (let x = 0; x < cow; ++x) {
          let s = cb[o];
          for (let c = 0; c < cc; ++c)
            for (let a = 0; a < k; ++a)
              for (let b = 0; b < k; ++b) {
                const iy = y * cs - cp + a, ix = x * cs - cp + b;
                if (iy >= 0 && iy < ch && ix >= 0 && ix < cw)
                  s += cx[((n * cc + c) * ch + iy) * cw + ix] * cwt[((o * cc + c) * k + a) * k + b];
              }
          cErr = Math.max(cErr, Math.abs(cy[((n * coc + o) * coh + y) * cow + x] - s));
        }
  out.conv_max_abs_err = cErr;
  ok = ok && cErr < 1e-5;

  // argmax over rows (first index on ties) and index_select of rows
  const ar = 5, ac = 37;
  const av = Float32Array.from({ length: ar * ac }, (_, i) => Math.round(8 * rnd()));
  const dav = upload(av), dai = hip.malloc(ar * 4);
  hip.argmax(dav.ptr, ar, ac, 1, 0, dai.ptr);
  const ai = await hip.d2hAsync(dai.ptr, new Int32Array(ar));
  let argOk = true;
  for (let r = 0; r < ar; ++r) {
    let best = 0;
    for (let c = 1; c < ac; ++c) if (av[r * ac + c] > av[r * ac + best]) best = c;
    argOk = argOk && ai[r] === best;
  }
  const sel = Int32Array.of(4, 0, 3, 2);
  const dsel = upload(sel), dso = hip.malloc(sel.length * ac * 4);
  hip.indexSelect(dav.ptr, 1, ar, ac, dsel.ptr, sel.length, dso.ptr);
  const so = await hip.d2hAsync(dso.ptr, new Float32Array(sel.length * ac));
  for (let j = 0; j < sel.length; ++j) {
    const row = sel[j];
    for (let c = 0; c < ac; ++c) argOk = argOk && so[j * ac + c] === av[row * ac + c];
  }
  out.argmax_index_select_exact = argOk;
  ok = ok && argOk;

  // d2hAsync copies in submission order: a fill launched right after the
  // call, and a free of the source, cannot change what the Promise returns
  const NS = 1 << 20;
  const src = Float32Array.from({ length: NS }, (_, i) => i % 977);
  const dsrc = upload(src);
  const pending = hip.d2hAsync(dsrc.ptr, new Float32Array(NS), dsrc);
  hip.fill(dsrc.ptr, NS, 7.0);
  const later = hip.d2hAsync(dsrc.ptr, new Float32Array(NS));
  hip.free(dsrc);
  const reuse = hip.malloc(NS * 4);  // the freed block, handed out again
  hip.fill(reuse.ptr, NS, -1.0);
  const [old, filled] = await Promise.all([pending, later]);
  let orderOk = true;
  for (let i = 0; i < NS; ++i) orderOk = orderOk && old[i] === src[i] && filled[i] === 7.0;
  out.d2h_async_submission_order = orderOk;
  ok = ok && orderOk;

  // free() then GC: the finalizer of a freed allocation must not return the
  // block again (it may belong to a newer allocation by then)
  if (typeof global.gc === 'function') {
    const blk = 1 << 16;
    let a = hip.malloc(blk);
    const pa = a.ptr;
    hip.free(a);
    let doubleFreeThrows = false;
    try { hip.free(a); } catch (e) { doubleFreeThrows = /already freed/.test(e.message); }
    a = null;
    const b = hip.malloc(blk);  // reuses the block `a` had
    global.gc();
    await new Promise((r) => setImmediate(r));
    global.gc();
    await new Promise((r) => setImmediate(r));
    const c = hip.malloc(blk);
    // b's block still belongs to b alone: c's writes do not reach it
    hip.fill(b.ptr, blk / 4, 1.0);
    hip.fill(c.ptr, blk / 4, 2.0);
    const bv = await hip.d2hAsync(b.ptr, new Float32Array(blk / 4), b);
    const intact = bv.every((v) => v === 1.0);
    const gcOk = b.ptr === pa && c.ptr !== b.ptr && doubleFreeThrows && intact;
    out.free_then_gc = { reused: b.ptr === pa, distinct: c.ptr !== b.ptr, doubleFreeThrows,
                         intact };
    ok = ok && gcOk;
    hip.free(b);
    hip.free(c);
  } else {
    out.free_then_gc = 'skipped (run node with --expose-gc)';
  }

  hip.synchronize();
  out.mem = hip.memoryStats();
  out.ok = ok;
  console.log(JSON.stringify(out));
  process.exit(ok ? 0 : 1);
}

main().catch((e) => {
  console.error(e && e.stack ? e.stack : e);
  process.exit(1);
});
