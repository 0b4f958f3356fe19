//! `HipTokenSampler`: AX Engine's `TokenSampler` plug-in
//! (crates/ax-engine-core/src/sampling.rs:90-92) on the MI355X sampler.
//!
//! Injected like any other sampler:
//! `EngineCore::with_runtime_components(kv, runner, Box::new(HipTokenSampler::new(0, 256, 262_144)?))`
//! (crates/ax-engine-core/src/engine.rs:165-176).
//!
//! Contract (the core `DeterministicSampler`'s, :97-136):
//! * one `SampledToken` per request, in order;
//! * invalid logits — empty, or a maximum under `f32::total_cmp` that is not
//!   finite (:172-178) — give token 0, `StopReason::Error`, no logprob;
//! * `MaxOutputTokens` when `generated_len + 1 >= max_output_tokens`;
//! * requests without logits keep the stub `previous_token + 1`, logprob 0.
//!
//! Requests with logits are sampled in one library call per vocabulary width
//! under the MLX law (`sample_categorical_into`,
//! crates/ax-engine-mlx/src/sampling.rs:204-316): greedy rows return the
//! first maximum with the core sampler's logprob (its sequential f32 sum
//! reproduced on the device); sampled rows draw with
//! Philox(seed, request_id, generated_len).  Ties keep the lowest id, where
//! `DeterministicSampler` keeps the last.  When the library fails, the batch
//! falls back to `DeterministicSampler`, as the runner's GPU helpers decline
//! to the CPU law (crates/ax-engine-mlx/src/generate.rs:221-238).
use std::fmt;

use ax_engine_core::sampling::{
    DeterministicSampler, SampledToken, SamplerInput, SamplerRequest, SamplingParams, StopReason,
    TokenSampler,
};
use hip_sys::philox::philox_uniform;
use hip_sys::{HipSamplerContext, HipSamplerError, HostBatch, RowParams};

const FLAG_ERROR: u32 = 1 << 31;

pub struct HipTokenSampler {
    ctx: HipSamplerContext,
    max_batch: usize,
    max_vocab: usize,
}

impl fmt::Debug for HipTokenSampler {
    fn fmt(&self, f: &mut fmt::Formatter<'_>) -> fmt::Result {
        f.debug_struct("HipTokenSampler")
            .field("device", &self.ctx.device())
            .field("max_batch", &self.max_batch)
            .field("max_vocab", &self.max_vocab)
            .finish()
    }
}

impl HipTokenSampler {
    pub fn new(device: i32, max_batch: usize, max_vocab: usize) -> Result<Self, HipSamplerError> {
        let ctx = HipSamplerContext::new(
            device,
            i32::try_from(max_batch).expect("max_batch fits in i32"),
            i32::try_from(max_vocab).expect("max_vocab fits in i32"),
        )?;
        Ok(Self { ctx, max_batch, max_vocab })
    }
}

/// The core sampler's validity test: the `total_cmp` maximum is finite.
fn logits_valid(logits: &[f32]) -> bool {
    logits
        .iter()
        .copied()
        .max_by(|a, b| a.total_cmp(b))
        .is_some_and(f32::is_finite)
}

fn row_params(p: &SamplingParams) -> RowParams {
    // Zeroed padding and extensions (presence / frequency: off).
    let mut r: RowParams = unsafe { std::mem::zeroed() };
    r.temperature = p.temperature;
    r.top_p = p.top_p;
    r.top_k = p.top_k;
    r.has_min_p = u32::from(p.min_p.is_some());
    r.min_p = p.min_p.unwrap_or(0.0);
    r.repetition_penalty = p.repetition_penalty;
    // the engine has already cut recent_tokens to the window
    // (crates/ax-engine-core/src/engine.rs:1180-1197); the core sampler
    // penalises all of them
    r.repetition_context_size = u32::MAX;
    r.no_repeat_ngram_size = p.no_repeat_ngram_size;
    r.ngram_window = p.ngram_window;
    r.presence_penalty = 0.0;
    r.frequency_penalty = 0.0;
    r.seed = p.seed;
    r.step = 0;
    r
}

impl HipTokenSampler {
    /// Samples the requests `idx` (all valid, all of width `vocab`) in one
    /// call; `None` when the library declines.
    fn sample_group(&self, reqs: &[SamplerRequest], idx: &[usize], vocab: usize) -> Option<Vec<(u32, f32, u32)>> {
        if vocab > self.max_vocab {
            return None;
        }
        let mut out = Vec::with_capacity(idx.len());
        for chunk in idx.chunks(self.max_batch.max(1)) {
            let mut logits = Vec::with_capacity(chunk.len() * vocab);
            let mut params = Vec::with_capacity(chunk.len());
            let mut history = Vec::new();
            let mut offsets = Vec::with_capacity(chunk.len() + 1);
            let mut uniforms = Vec::with_capacity(chunk.len());
            offsets.push(0i64);
            for &i in chunk {
                let rq = &reqs[i];
                logits.extend_from_slice(rq.logits.as_deref().unwrap_or(&[]));
                params.push(row_params(&rq.sampling_params));
                history.extend_from_slice(&rq.recent_tokens);
                offsets.push(history.len() as i64);
                uniforms.push(philox_uniform(
                    rq.sampling_params.seed,
                    rq.request_id.0 as u32,
                    u64::from(rq.generated_len),
                ));
            }
            let batch = HostBatch {
                logits: &logits,
                batch: chunk.len(),
                vocab,
                params: &params,
                history: &history,
                history_offsets: &offsets,
                uniforms: Some(&uniforms),
            };
            let res = self.ctx.sample_host(&batch, true).ok()?;
            for k in 0..chunk.len() {
                out.push((res.token_ids[k], res.logprobs[k], res.flags[k]));
            }
        }
        Some(out)
    }
}

impl TokenSampler for HipTokenSampler {
    fn sample(&self, input: SamplerInput) -> Vec<SampledToken> {
        let reqs = input.requests;
        // (token, logprob) of each request sampled on the GPU
        let mut sampled: Vec<Option<(u32, f32)>> = vec![None; reqs.len()];
        let mut widths: Vec<usize> = Vec::new();
        for rq in &reqs {
            if let Some(l) = &rq.logits {
                if logits_valid(l) && !widths.contains(&l.len()) {
                    widths.push(l.len());
                }
            }
        }
        for vocab in widths {
            let idx: Vec<usize> = reqs
                .iter()
                .enumerate()
                .filter(|(_, rq)| rq.logits.as_ref().is_some_and(|l| l.len() == vocab && logits_valid(l)))
                .map(|(i, _)| i)
                .collect();
            match self.sample_group(&reqs, &idx, vocab) {
                Some(rows) => {
                    for (&i, (tok, lp, flags)) in idx.iter().zip(rows) {
                        if flags & FLAG_ERROR == 0 {
                            sampled[i] = Some((tok, lp));
                        }
                    }
                }
                None => {
                    // the library declined: these requests take the CPU law
                    let cpu = DeterministicSampler.sample(SamplerInput {
                        requests: idx.iter().map(|&i| reqs[i].clone()).collect(),
                    });
                    for (&i, t) in idx.iter().zip(cpu) {
                        if let Some(lp) = t.logprob {
                            sampled[i] = Some((t.token_id, lp));
                        }
                    }
                }
            }
        }
        reqs.iter()
            .zip(sampled)
            .map(|(rq, s)| {
                let invalid = rq.logits.is_some() && s.is_none();
                let (token_id, logprob) = match (invalid, s) {
                    (true, _) => (0, None),
                    (false, Some((t, lp))) => (t, Some(lp)),
                    (false, None) => (rq.previous_token.saturating_add(1), Some(0.0)),
                };
                let stop_reason = if invalid {
                    Some(StopReason::Error)
                } else if rq.generated_len.saturating_add(1) >= rq.max_output_tokens {
                    Some(StopReason::MaxOutputTokens)
                } else {
                    None
                };
                SampledToken { request_id: rq.request_id, token_id, stop_reason, logprob }
            })
            .collect()
    }
}
