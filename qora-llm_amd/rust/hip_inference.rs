//! `src/hip_inference.rs` of the reference crate, behind its `hip` feature:
//! the device-resident counterpart of the CPU pair
//!   raw_prefill(&DecodeWeights, &[u32]) -> (Vec<f32>, RawKvCache)   (gemv.rs:1027)
//!   forward_decode_raw(&DecodeWeights, usize, &mut RawKvCache)      (gemv.rs:872)
//! over libqora_hip.so through the qora-hip-sys crate. The KV cache lives in
//! the device context instead of a RawKvCache. Every failure is an Err
//! string, so the caller keeps main.rs's fall back to the CPU path
//! (main.rs:143-151). Needs the crate's `WeightRef` / `layer_ref` /
//! `embed_ref` views (gemv.rs:65-96, 245-271), which the `hip` feature
//! enables alongside `gpu` and `gpu-metal`.

use std::ffi::CStr;

use qora_hip_sys as sys;

use crate::gemv::{DecodeWeights, WeightRef};

pub use sys::qora_sample_params as SampleParams;

pub struct HipDecoder {
    ctx: *mut sys::qora_hip_ctx,
    vocab: usize,
}

fn err(ctx: *mut sys::qora_hip_ctx, what: &str) -> String {
    let msg = unsafe { CStr::from_ptr(sys::qora_hip_last_error(ctx)) };
    format!("{what}: {}", msg.to_string_lossy())
}

fn upload(ctx: *mut sys::qora_hip_ctx, w: &WeightRef) -> Result<u32, String> {
    let mut id = 0u32;
    let rc = unsafe {
        match w {
            WeightRef::Q4 { packed, scales, k, n } => sys::qora_hip_upload_q4(
                ctx,
                packed.as_ptr(),
                packed.len(),
                scales.as_ptr() as *const u16,
                scales.len(),
                *k as u64,
                *n as u64,
                &mut id,
            ),
            WeightRef::F16 { data, k, n } => {
                sys::qora_hip_upload_f16(ctx, data.as_ptr() as *const u16, data.len(), *k as u64, *n as u64, &mut id)
            }
        }
    };
    if rc != sys::QORA_HIP_OK {
        Err(err(ctx, "upload"))
    } else {
        Ok(id)
    }
}

impl HipDecoder {
    /// Uploads the weights and sets the model up with a device cache of
    /// `kv_capacity` positions (0: the RoPE table's length). generate_hip
    /// passes prompt length + max_new_tokens + 1: the device cache does not
    /// grow, and a step past it returns QORA_HIP_E_STATE.
    pub fn new(w: &DecodeWeights, kv_capacity: u32) -> Result<Self, String> {
        let mut ctx = std::ptr::null_mut();
        if unsafe { sys::qora_hip_create(0, &mut ctx) } != sys::QORA_HIP_OK {
            return Err("no HIP device".into());
        }
        // Drop destroys the context on any error below
        let me = HipDecoder { ctx, vocab: w.vocab() };
        let nl = w.num_layers();
        let (mut wids, mut g1, mut g2) = (Vec::with_capacity(nl * 7), Vec::new(), Vec::new());
        let mut heads = (0, 0, 0, 0);
        let mut inter = 0;
        for i in 0..nl {
            let l = w.layer_ref(i);
            for r in [&l.q_proj, &l.k_proj, &l.v_proj, &l.o_proj, &l.gate_proj, &l.up_proj, &l.down_proj] {
                wids.push(upload(ctx, r)?);
            }
            if let WeightRef::Q4 { n, .. } | WeightRef::F16 { n, .. } = &l.gate_proj {
                inter = *n;
            }
            g1.push(l.input_norm_gamma.as_ptr() as *const u16);
            g2.push(l.post_attn_norm_gamma.as_ptr() as *const u16);
            heads = (l.num_heads, l.num_kv_heads, l.head_dim, l.num_kv_groups);
        }
        let embed_wid = upload(ctx, &w.embed_ref())?;
        let use_rope: Vec<u8> = w.no_rope_layers_ref().iter().map(|&b| b as u8).collect();
        let half = w.rope_half_dim();
        let desc = sys::qora_model_desc {
            num_layers: nl as u32,
            vocab: w.vocab() as u32,
            hidden: w.hidden() as u32,
            intermediate: inter as u32,
            num_heads: heads.0 as u32,
            num_kv_heads: heads.1 as u32,
            head_dim: heads.2 as u32,
            num_kv_groups: heads.3 as u32,
            rope_half_dim: half as u32,
            format: w.format_id() as u32,
            layer_wids: wids.as_ptr(),
            input_norm: g1.as_ptr(),
            post_attn_norm: g2.as_ptr(),
            embed_wid,
            final_norm: w.final_norm_ref().as_ptr() as *const u16,
            rope_cos: w.rope_cos_ref().as_ptr(),
            rope_sin: w.rope_sin_ref().as_ptr(),
            rope_positions: (w.rope_cos_ref().len() / half.max(1)) as u64,
            use_rope: use_rope.as_ptr(),
            kv_capacity,
            kv_dtype: 0,
        };
        if unsafe { sys::qora_hip_model_init(ctx, &desc) } != sys::QORA_HIP_OK {
            return Err(err(ctx, "model_init"));
        }
        Ok(me)
    }

    /// raw_prefill: resets the device cache, returns the last position's logits.
    pub fn prefill(&mut self, ids: &[u32]) -> Result<Vec<f32>, String> {
        let mut logits = vec![0f32; self.vocab];
        let rc = unsafe {
            sys::qora_hip_prefill(self.ctx, ids.as_ptr(), ids.len(), logits.as_mut_ptr(), std::ptr::null_mut())
        };
        if rc != sys::QORA_HIP_OK {
            Err(err(self.ctx, "prefill"))
        } else {
            Ok(logits)
        }
    }

    /// forward_decode_raw: one token at the current cache position.
    pub fn decode(&mut self, token: usize) -> Result<Vec<f32>, String> {
        let mut logits = vec![0f32; self.vocab];
        let rc = unsafe { sys::qora_hip_decode(self.ctx, token as u32, logits.as_mut_ptr(), std::ptr::null_mut()) };
        if rc != sys::QORA_HIP_OK {
            Err(err(self.ctx, "decode"))
        } else {
            Ok(logits)
        }
    }

    /// Greedy step without the logits copy: only the first-max token
    /// (sample_token_top_k's greedy branch, generate.rs:346-352) comes back.
    pub fn decode_greedy(&mut self, token: usize) -> Result<u32, String> {
        let mut next = 0u32;
        let rc = unsafe { sys::qora_hip_decode(self.ctx, token as u32, std::ptr::null_mut(), &mut next) };
        if rc != sys::QORA_HIP_OK {
            Err(err(self.ctx, "decode"))
        } else {
            Ok(next)
        }
    }

    /// Sampled step: the decode step, the penalties and sample_token_top_k on
    /// the device (generate.rs:64-91, 345-395); `rng` is the Rng state, which
    /// the call advances as the reference's draws do.
    pub fn decode_sample(&mut self, token: usize, generated: &[u32], p: &SampleParams, rng: &mut u64)
                         -> Result<u32, String> {
        let mut next = 0u32;
        let rc = unsafe {
            sys::qora_hip_decode_sample(self.ctx, token as u32, generated.as_ptr(), generated.len() as u64, p, rng,
                                        std::ptr::null_mut(), &mut next)
        };
        if rc != sys::QORA_HIP_OK {
            Err(err(self.ctx, "decode_sample"))
        } else {
            Ok(next)
        }
    }

    /// A caller-built RawKvCache (gemv.rs:154-166) handed to the device: every
    /// layer's (k, v, len), all with the same length.
    pub fn load_cache(&mut self, cache: &[(Vec<f32>, Vec<f32>, usize)]) -> Result<(), String> {
        for (i, (k, v, len)) in cache.iter().enumerate() {
            let rc = unsafe { sys::qora_hip_kv_upload(self.ctx, i as u32, k.as_ptr(), v.as_ptr(), *len as u64) };
            if rc != sys::QORA_HIP_OK {
                return Err(err(self.ctx, "kv_upload"));
            }
        }
        Ok(())
    }
}

impl Drop for HipDecoder {
    fn drop(&mut self) {
        unsafe {
            sys::qora_hip_destroy(self.ctx);
        }
    }
}
