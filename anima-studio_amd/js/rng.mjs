// torch.randn on the CPU generator (app/rng.js:1-67), so that a seed gives the initial noise and
// the ancestral / SDE noise of ComfyUI (torch.manual_seed(seed); torch.randn(n)).  The stream is
// MT19937; torch's float normal fill turns each block of 16 uniforms (24 random bits each) into 8
// Box-Muller pairs.  Every intermediate is rounded to float where the reference rounds it
// (Math.fround), so the values equal the reference's bit for bit.

const N = 624;

class MersenneTwister {
  constructor(seed) {
    this.s = new Uint32Array(N);
    this.s[0] = Number(BigInt.asUintN(32, BigInt(seed)));
    for (let i = 1; i < N; i++) {
      const p = this.s[i - 1] ^ (this.s[i - 1] >>> 30);
      this.s[i] = (Math.imul(1812433253, p) + i) >>> 0;
    }
    this.pos = N;
  }

  // regenerate the whole state (in place, in index order)
  regen() {
    const s = this.s;
    for (let i = 0; i < N; i++) {
      const y = (s[i] & 0x80000000) | (s[(i + 1) % N] & 0x7fffffff);
      s[i] = (s[(i + 397) % N] ^ (y >>> 1) ^ (y & 1 ? 0x9908b0df : 0)) >>> 0;
    }
    this.pos = 0;
  }

  u32() {
    if (this.pos >= N) this.regen();
    let y = this.s[this.pos++];
    y ^= y >>> 11;
    y ^= (y << 7) & 0x9d2c5680;
    y ^= (y << 15) & 0xefc60000;
    y ^= y >>> 18;
    return y >>> 0;
  }
}

export class TorchGenerator {
  constructor(seed) {
    this.mt = new MersenneTwister(seed);
  }

  // uniform float in [0, 1) from the low 24 bits
  uniform() {
    return Math.fround((this.mt.u32() & 0xffffff) / 16777216);
  }

  // Box-Muller over d[o .. o+15]: pairs (j, j + 8)
  static boxMuller16(d, o) {
    const f = Math.fround;
    for (let j = 0; j < 8; j++) {
      const u1 = f(1 - d[o + j]);
      const u2 = d[o + j + 8];
      const radius = f(Math.sqrt(f(-2 * f(Math.log(u1)))));
      const theta = f(2.0 * Math.PI * u2);
      d[o + j] = f(radius * f(Math.cos(theta)));
      d[o + j + 8] = f(radius * f(Math.sin(theta)));
    }
  }

  // torch.randn(n) in float32, n >= 16: n uniforms, Box-Muller per block of 16, and for a ragged
  // tail 16 fresh uniforms over the last 16 slots
  randn(n) {
    if (n < 16) throw new Error("randn: n must be at least 16");
    const d = new Float32Array(n);
    for (let i = 0; i < n; i++) d[i] = this.uniform();
    for (let i = 0; i + 16 <= n; i += 16) TorchGenerator.boxMuller16(d, i);
    if (n % 16) {
      const o = n - 16;
      for (let i = 0; i < 16; i++) d[o + i] = this.uniform();
      TorchGenerator.boxMuller16(d, o);
    }
    return d;
  }
}
