// Host-side tables and layout helpers of the DiT (no GPU compute here).
// Restates app/models/common.js (RoPE tables) and app/models/dit.js:41-78 (timestep embedding,
// patchify / unpatchify).

const D = 2048;

// cos block followed by sin block, each [L][half]; returned Tensor carries .sinOff
// (app/models/common.js:3-12).
export function ropeTableTensor(gpu, angles, L, half) {
  const cs = new Float32Array(2 * L * half);
  for (let i = 0; i < L * half; i++) {
    cs[i] = Math.cos(angles[i]);
    cs[L * half + i] = Math.sin(angles[i]);
  }
  const t = gpu.fromArray(cs, [cs.length]);
  t.sinOff = L * half;
  return t;
}

// Standard 1D rope of the text encoder: angle(l, i) = l * fround(1 / theta^(2i / D))
// (app/models/common.js:15-22).
export function ropeTable(gpu, L, Dh, theta) {
  const half = Dh / 2;
  const a = new Float32Array(L * half);
  for (let l = 0; l < L; l++) {
    for (let i = 0; i < half; i++) a[l * half + i] = l * Math.fround(1 / Math.pow(theta, (2 * i) / Dh));
  }
  return ropeTableTensor(gpu, a, L, half);
}

// Cosmos VideoRopePosition3DEmb for one frame: 64 slots = 22 temporal (position 0), 21 height,
// 21 width, NTK-scaled theta for h/w (app/models/common.js:31-52).
export function ditRopeAngles(H, W) {
  const headDim = 128;
  const dimH = Math.floor(headDim / 6) * 2; // 42
  const dimT = headDim - 2 * dimH; // 44
  const hTheta = 10000 * Math.pow(4, dimH / (dimH - 2));
  const hf = [];
  for (let j = 0; j < dimH / 2; j++) hf.push(Math.fround(1 / Math.pow(hTheta, Math.fround((2 * j) / dimH))));
  const half = 64;
  const a = new Float32Array(H * W * half);
  for (let y = 0; y < H; y++) {
    for (let x = 0; x < W; x++) {
      const o = (y * W + x) * half;
      for (let j = 0; j < 21; j++) {
        a[o + dimT / 2 + j] = y * hf[j];
        a[o + dimT / 2 + 21 + j] = x * hf[j];
      }
    }
  }
  return a;
}

export function ditRopeTable(gpu, H, W) {
  return ropeTableTensor(gpu, ditRopeAngles(H, W), H * W, 64);
}

// Sinusoidal timestep embedding [D]: cos half then sin half (app/models/dit.js:41-51).
export function timestepEmbedding(sigma) {
  const half = D / 2;
  const temb = new Float32Array(D);
  for (let i = 0; i < half; i++) {
    const f = Math.fround(Math.exp(Math.fround((-Math.log(10000) * i) / half)));
    const a = Math.fround(sigma * f);
    temb[i] = Math.cos(a);
    temb[half + i] = Math.sin(a);
  }
  return temb;
}

// latent [16, h, w] -> patches [(h/2)(w/2), 68], "c (h m) (w n) -> (h w) (c m n)" with the zero
// padding-mask channel c = 16 (app/models/dit.js:55-65).  Writes into `out` at `offset`.
export function patchify(latent, h, w, out, offset) {
  const Hp = h / 2, Wp = w / 2;
  const patches = out || new Float32Array(Hp * Wp * 68);
  const base = offset || 0;
  for (let y = 0; y < Hp; y++) for (let x = 0; x < Wp; x++) {
    const o = base + (y * Wp + x) * 68;
    for (let c = 0; c < 16; c++) for (let m = 0; m < 2; m++) for (let n = 0; n < 2; n++) {
      patches[o + c * 4 + m * 2 + n] = latent[c * h * w + (2 * y + m) * w + (2 * x + n)];
    }
    for (let k = 64; k < 68; k++) patches[o + k] = 0;
  }
  return patches;
}

// final layer output [(h/2)(w/2), 64] -> [16, h, w], "(h w) (p1 p2 c) -> c (h p1) (w p2)"
// (app/models/dit.js:68-78).  Reads `o` from `offset`.
export function unpatchify(o, h, w, offset) {
  const Hp = h / 2, Wp = w / 2;
  const base = offset || 0;
  const v = new Float32Array(16 * h * w);
  for (let y = 0; y < Hp; y++) for (let xx = 0; xx < Wp; xx++) {
    const b = base + (y * Wp + xx) * 64;
    for (let p1 = 0; p1 < 2; p1++) for (let p2 = 0; p2 < 2; p2++) for (let c = 0; c < 16; c++) {
      v[c * h * w + (2 * y + p1) * w + (2 * xx + p2)] = o[b + p1 * 32 + p2 * 16 + c];
    }
  }
  return v;
}
