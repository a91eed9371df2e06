from fused_decode.bench import main

if __name__ == "__main__":
    main()
